/*
 * oracle.c -- CPU restatement of the reference's fp32 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY: see oracle.h.  Built with gcc -O2
 * -ffp-contract=off so every multiply and add rounds separately, as the
 * reference's host loops do on x86-64 without FMA.
 */
#include "oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum { EPI_NONE = 0, EPI_BIAS = 1, EPI_BIAS_RELU = 2, EPI_RELU = 3, EPI_RELU_GRAD = 4 };

void oracle_gemm_cpu_rows(const float* a, const float* b, float* c, size_t m, size_t n,
                          size_t k, size_t row0, size_t row1) {
    (void)m;
    for (size_t row = row0; row < row1; ++row) {
        for (size_t col = 0; col < n; ++col) {
            float sum = 0.0f;
            for (size_t kk = 0; kk < k; ++kk) {
                sum += a[row * k + kk] * b[kk * n + col];
            }
            c[row * n + col] = sum;
        }
    }
}

void oracle_gemm_cpu(const float* a, const float* b, float* c, size_t m, size_t n, size_t k) {
    oracle_gemm_cpu_rows(a, b, c, m, n, k, 0, m);
}

static inline float op_a(int ta, const float* A, int64_t lda, int64_t i, int64_t k) {
    return ta ? A[k * lda + i] : A[i * lda + k];
}

static inline float op_b(int tb, const float* B, int64_t ldb, int64_t k, int64_t j) {
    return tb ? B[j * ldb + k] : B[k * ldb + j];
}

/* std::max(0.0f, v) == (0 < v) ? v : 0 */
static inline float relu_f(float v) { return (0.0f < v) ? v : 0.0f; }
static inline double relu_d(double v) { return (0.0 < v) ? v : 0.0; }

void oracle_sgemm_ex(int transA, int transB, int64_t M, int64_t N, int64_t K,
                     const float* A, int64_t lda, int64_t strideA,
                     const float* B, int64_t ldb, int64_t strideB,
                     float* C, int64_t ldc, int64_t strideC, int64_t batch,
                     const float* bias, const float* aux, int epilogue) {
    for (int64_t bz = 0; bz < batch; ++bz) {
        const float* Ab = A + bz * strideA;
        const float* Bb = B + bz * strideB;
        float* Cb = C + bz * strideC;
        const float* Xb = aux ? aux + bz * strideC : NULL;
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) {
                float sum = 0.0f;
                for (int64_t k = 0; k < K; ++k) {
                    sum += op_a(transA, Ab, lda, i, k) * op_b(transB, Bb, ldb, k, j);
                }
                float v = sum;
                switch (epilogue) {
                    case EPI_BIAS: v = sum + bias[j]; break;
                    case EPI_BIAS_RELU: v = relu_f(sum + bias[j]); break;
                    case EPI_RELU: v = relu_f(sum); break;
                    case EPI_RELU_GRAD: v = Xb[i * ldc + j] > 0.0f ? sum : 0.0f; break;
                    default: break;
                }
                Cb[i * ldc + j] = v;
            }
        }
    }
}

void oracle_sgemm_ex_f64(int transA, int transB, int64_t M, int64_t N, int64_t K,
                         const float* A, int64_t lda, int64_t strideA,
                         const float* B, int64_t ldb, int64_t strideB,
                         double* C64, double* ABS64, int64_t ldc, int64_t strideC,
                         int64_t batch, const float* bias, const float* aux, int epilogue) {
    for (int64_t bz = 0; bz < batch; ++bz) {
        const float* Ab = A + bz * strideA;
        const float* Bb = B + bz * strideB;
        const float* Xb = aux ? aux + bz * strideC : NULL;
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) {
                double sum = 0.0, asum = 0.0;
                for (int64_t k = 0; k < K; ++k) {
                    const double x = op_a(transA, Ab, lda, i, k);
                    const double y = op_b(transB, Bb, ldb, k, j);
                    sum += x * y;
                    asum += fabs(x) * fabs(y);
                }
                double v = sum;
                switch (epilogue) {
                    case EPI_BIAS: v = sum + bias[j]; asum += fabs((double)bias[j]); break;
                    case EPI_BIAS_RELU: v = relu_d(sum + bias[j]); asum += fabs((double)bias[j]); break;
                    case EPI_RELU: v = relu_d(sum); break;
                    case EPI_RELU_GRAD: v = Xb[i * ldc + j] > 0.0f ? sum : 0.0; break;
                    default: break;
                }
                const int64_t off = bz * strideC + i * ldc + j;
                C64[off] = v;
                if (ABS64) ABS64[off] = asum;
            }
        }
    }
}

void oracle_linear(const float* x, const float* w, const float* bias, float* y,
                   size_t batch, size_t in_features, size_t out_features) {
    for (size_t row = 0; row < batch; ++row) {
        for (size_t col = 0; col < out_features; ++col) {
            float sum = 0.0f;
            for (size_t k = 0; k < in_features; ++k) {
                sum += x[row * in_features + k] * w[k * out_features + col];
            }
            y[row * out_features + col] = sum + bias[col];
        }
    }
}

void oracle_relu(const float* x, float* y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = relu_f(x[i]);
}

void oracle_relu_backward(const float* g, const float* act, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = act[i] > 0.0f ? g[i] : 0.0f;
}

void oracle_colsum(const float* x, float* out, size_t rows, size_t cols) {
    for (size_t c = 0; c < cols; ++c) {
        float s = 0.0f;
        for (size_t r = 0; r < rows; ++r) s += x[r * cols + c];
        out[c] = s;
    }
}

void oracle_softmax(const float* x, float* y, size_t rows, size_t cols) {
    for (size_t row = 0; row < rows; ++row) {
        const size_t off = row * cols;
        float mx = x[off];
        for (size_t c = 1; c < cols; ++c) mx = x[off + c] > mx ? x[off + c] : mx;
        float sum = 0.0f;
        for (size_t c = 0; c < cols; ++c) {
            const float v = expf(x[off + c] - mx);
            y[off + c] = v;
            sum += v;
        }
        for (size_t c = 0; c < cols; ++c) y[off + c] /= sum;
    }
}

float oracle_cross_entropy(const float* logits, const int64_t* labels, size_t batch,
                           size_t classes) {
    float loss = 0.0f;
    for (size_t row = 0; row < batch; ++row) {
        const int64_t label = labels[row];
        if (label < 0 || label >= (int64_t)classes) continue;
        const size_t off = row * classes;
        float mx = logits[off];
        for (size_t c = 1; c < classes; ++c) mx = logits[off + c] > mx ? logits[off + c] : mx;
        float sum_exp = 0.0f;
        for (size_t c = 0; c < classes; ++c) sum_exp += expf(logits[off + c] - mx);
        loss += logf(sum_exp) + mx - logits[off + (size_t)label];
    }
    return loss / (float)batch;
}

void oracle_softmax_xent_grad(const float* logits, const int64_t* labels, float* grad,
                              size_t batch, size_t classes) {
    oracle_softmax(logits, grad, batch, classes);
    for (size_t row = 0; row < batch; ++row) {
        const int64_t y = labels[row];
        if (y >= 0 && y < (int64_t)classes) grad[row * classes + (size_t)y] -= 1.0f;
    }
    for (size_t i = 0; i < batch * classes; ++i) grad[i] /= (float)batch;
}

void oracle_sgd(float* p, const float* g, float lr, size_t n) {
    for (size_t i = 0; i < n; ++i) p[i] -= lr * g[i];
}

void oracle_mlp2_train_step(const float* X, const int64_t* labels, int64_t batch,
                            int64_t in_features, int64_t hidden, int64_t classes,
                            float* W1, float* b1, float* W2, float* b2, float lr,
                            float* H, float* logits, float* G2, float* G1,
                            float* dW1, float* db1, float* dW2, float* db2,
                            float* dX, float* loss) {
    const int64_t B = batch, I = in_features, Hd = hidden, Cc = classes;
    /* forward (Network.cpp:7-14) */
    oracle_sgemm_ex(0, 0, B, Hd, I, X, I, 0, W1, Hd, 0, H, Hd, 0, 1, b1, NULL, EPI_BIAS_RELU);
    oracle_sgemm_ex(0, 0, B, Cc, Hd, H, Hd, 0, W2, Cc, 0, logits, Cc, 0, 1, b2, NULL, EPI_BIAS);
    /* loss and its gradient (Network.cpp:16-22) */
    *loss = oracle_cross_entropy(logits, labels, (size_t)B, (size_t)Cc);
    oracle_softmax_xent_grad(logits, labels, G2, (size_t)B, (size_t)Cc);
    /* backward through layer 2, ReLU, layer 1 (Network.cpp:23-25, Layers.cpp:36-44) */
    oracle_sgemm_ex(1, 0, Hd, Cc, B, H, Hd, 0, G2, Cc, 0, dW2, Cc, 0, 1, NULL, NULL, EPI_NONE);
    oracle_colsum(G2, db2, (size_t)B, (size_t)Cc);
    oracle_sgemm_ex(0, 1, B, Hd, Cc, G2, Cc, 0, W2, Cc, 0, G1, Hd, 0, 1, NULL, H, EPI_RELU_GRAD);
    oracle_sgemm_ex(1, 0, I, Hd, B, X, I, 0, G1, Hd, 0, dW1, Hd, 0, 1, NULL, NULL, EPI_NONE);
    oracle_colsum(G1, db1, (size_t)B, (size_t)Hd);
    if (dX) {
        oracle_sgemm_ex(0, 1, B, I, Hd, G1, Hd, 0, W1, Hd, 0, dX, I, 0, 1, NULL, NULL, EPI_NONE);
    }
    /* update (Network.cpp:29-34, Optimizer.hpp:24-34) */
    oracle_sgd(W1, dW1, lr, (size_t)(I * Hd));
    oracle_sgd(b1, db1, lr, (size_t)Hd);
    oracle_sgd(W2, dW2, lr, (size_t)(Hd * Cc));
    oracle_sgd(b2, db2, lr, (size_t)Cc);
}

/* fp64 forward of the MLP; returns the loss and (optionally) keeps Z1, H, P. */
static double mlp2_forward_f64(const double* X, const int64_t* labels, int64_t B, int64_t I,
                               int64_t Hd, int64_t Cc, const double* W1, const double* b1,
                               const double* W2, const double* b2, double* Z1, double* Hh,
                               double* P) {
    for (int64_t r = 0; r < B; ++r) {
        for (int64_t h = 0; h < Hd; ++h) {
            double s = 0.0;
            for (int64_t i = 0; i < I; ++i) s += X[r * I + i] * W1[i * Hd + h];
            s += b1[h];
            Z1[r * Hd + h] = s;
            Hh[r * Hd + h] = relu_d(s);
        }
    }
    double loss = 0.0;
    for (int64_t r = 0; r < B; ++r) {
        double* z = P + r * Cc;
        for (int64_t c = 0; c < Cc; ++c) {
            double s = 0.0;
            for (int64_t h = 0; h < Hd; ++h) s += Hh[r * Hd + h] * W2[h * Cc + c];
            z[c] = s + b2[c];
        }
        double mx = z[0];
        for (int64_t c = 1; c < Cc; ++c) mx = z[c] > mx ? z[c] : mx;
        double se = 0.0;
        for (int64_t c = 0; c < Cc; ++c) se += exp(z[c] - mx);
        const int64_t y = labels[r];
        if (y >= 0 && y < Cc) loss += log(se) + mx - z[y];
        for (int64_t c = 0; c < Cc; ++c) z[c] = exp(z[c] - mx) / se;
    }
    return loss / (double)B;
}

double oracle_mlp2_loss_f64(const double* X, const int64_t* labels, int64_t batch,
                            int64_t in_features, int64_t hidden, int64_t classes,
                            const double* W1, const double* b1, const double* W2,
                            const double* b2) {
    double* Z1 = (double*)malloc(sizeof(double) * (size_t)(batch * hidden));
    double* Hh = (double*)malloc(sizeof(double) * (size_t)(batch * hidden));
    double* P = (double*)malloc(sizeof(double) * (size_t)(batch * classes));
    const double loss = mlp2_forward_f64(X, labels, batch, in_features, hidden, classes, W1, b1,
                                         W2, b2, Z1, Hh, P);
    free(Z1);
    free(Hh);
    free(P);
    return loss;
}

void oracle_mlp2_grads_f64(const double* X, const int64_t* labels, int64_t batch,
                           int64_t in_features, int64_t hidden, int64_t classes,
                           const double* W1, const double* b1, const double* W2,
                           const double* b2, double* dW1, double* db1, double* dW2,
                           double* db2, double* dX) {
    const int64_t B = batch, I = in_features, Hd = hidden, Cc = classes;
    double* Z1 = (double*)malloc(sizeof(double) * (size_t)(B * Hd));
    double* Hh = (double*)malloc(sizeof(double) * (size_t)(B * Hd));
    double* P = (double*)malloc(sizeof(double) * (size_t)(B * Cc));
    double* G1 = (double*)malloc(sizeof(double) * (size_t)(B * Hd));
    mlp2_forward_f64(X, labels, B, I, Hd, Cc, W1, b1, W2, b2, Z1, Hh, P);
    /* G2 = (P - onehot) / B, stored in P */
    for (int64_t r = 0; r < B; ++r) {
        const int64_t y = labels[r];
        if (y >= 0 && y < Cc) P[r * Cc + y] -= 1.0;
        for (int64_t c = 0; c < Cc; ++c) P[r * Cc + c] /= (double)B;
    }
    for (int64_t h = 0; h < Hd; ++h)
        for (int64_t c = 0; c < Cc; ++c) {
            double s = 0.0;
            for (int64_t r = 0; r < B; ++r) s += Hh[r * Hd + h] * P[r * Cc + c];
            dW2[h * Cc + c] = s;
        }
    for (int64_t c = 0; c < Cc; ++c) {
        double s = 0.0;
        for (int64_t r = 0; r < B; ++r) s += P[r * Cc + c];
        db2[c] = s;
    }
    for (int64_t r = 0; r < B; ++r)
        for (int64_t h = 0; h < Hd; ++h) {
            double s = 0.0;
            for (int64_t c = 0; c < Cc; ++c) s += P[r * Cc + c] * W2[h * Cc + c];
            G1[r * Hd + h] = Z1[r * Hd + h] > 0.0 ? s : 0.0;
        }
    for (int64_t i = 0; i < I; ++i)
        for (int64_t h = 0; h < Hd; ++h) {
            double s = 0.0;
            for (int64_t r = 0; r < B; ++r) s += X[r * I + i] * G1[r * Hd + h];
            dW1[i * Hd + h] = s;
        }
    for (int64_t h = 0; h < Hd; ++h) {
        double s = 0.0;
        for (int64_t r = 0; r < B; ++r) s += G1[r * Hd + h];
        db1[h] = s;
    }
    if (dX) {
        for (int64_t r = 0; r < B; ++r)
            for (int64_t i = 0; i < I; ++i) {
                double s = 0.0;
                for (int64_t h = 0; h < Hd; ++h) s += G1[r * Hd + h] * W1[i * Hd + h];
                dX[r * I + i] = s;
            }
    }
    free(Z1);
    free(Hh);
    free(P);
    free(G1);
}

/* ------------------------------------------------------------ IDX files */

/* to_int, legacy/src/data/DataLoader.cpp:22-25. */
static int idx_word(FILE* f, int64_t* out) {
    unsigned char p[4];
    if (fread(p, 1, 4, f) != 4) return -3;
    const uint32_t v = ((uint32_t)p[0] << 24) | ((uint32_t)p[1] << 16) | ((uint32_t)p[2] << 8) |
                       (uint32_t)p[3];
    *out = (int64_t)(int32_t)v;
    return 0;
}

/* The num limit, DataLoader.cpp:43,85. */
static int64_t idx_limit(int64_t count, int64_t num) {
    return (num != 0 && num < count) ? num : count;
}

int oracle_idx_read_images(const char* path, int64_t num, int64_t* count, int64_t* rows,
                           int64_t* cols, float* images) {
    if (num < 0) return -4;
    FILE* f = fopen(path, "rb");
    if (!f) return -1;
    int64_t magic = 0, n = 0, r = 0, c = 0;
    int rc = idx_word(f, &magic);
    if (rc == 0 && magic != 0x803) rc = -2;
    if (rc == 0) rc = idx_word(f, &n);
    if (rc == 0) rc = idx_word(f, &r);
    if (rc == 0) rc = idx_word(f, &c);
    if (rc == 0 && (n < 0 || r < 0 || c < 0)) rc = -4;
    if (rc == 0) {
        n = idx_limit(n, num);
        *count = n;
        *rows = r;
        *cols = c;
        if (images) {
            const int64_t size = r * c;
            unsigned char* q = (unsigned char*)malloc(size > 0 ? (size_t)size : 1);
            for (int64_t i = 0; i < n && rc == 0; ++i) {
                if ((int64_t)fread(q, 1, (size_t)size, f) != size) {
                    rc = -3;
                    break;
                }
                /* DataLoader.cpp:64-67 */
                for (int64_t j = 0; j < size; ++j) images[i * size + j] = (float)q[j] / 255.0f;
            }
            free(q);
        }
    }
    fclose(f);
    return rc;
}

int oracle_idx_read_labels(const char* path, int64_t num, int64_t* count, int64_t* labels) {
    if (num < 0) return -4;
    FILE* f = fopen(path, "rb");
    if (!f) return -1;
    int64_t magic = 0, n = 0;
    int rc = idx_word(f, &magic);
    if (rc == 0 && magic != 0x801) rc = -2;
    if (rc == 0) rc = idx_word(f, &n);
    if (rc == 0 && n < 0) rc = -4;
    if (rc == 0) {
        n = idx_limit(n, num);
        *count = n;
        for (int64_t i = 0; labels && i < n; ++i) {
            signed char p;
            if (fread(&p, 1, 1, f) != 1) {
                rc = -3;
                break;
            }
            labels[i] = (int64_t)p; /* DataLoader.cpp:88-90: int label = p[0] (char) */
        }
    }
    fclose(f);
    return rc;
}

void oracle_idx_gather(const uint8_t* images, const uint8_t* labels, int64_t count,
                       int64_t row_bytes, const int64_t* index, int64_t batch, float divisor,
                       float* x, int64_t* y) {
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t r = index ? index[b] : b;
        const int ok = r >= 0 && r < count;
        for (int64_t j = 0; x && j < row_bytes; ++j) {
            x[b * row_bytes + j] = ok ? (float)images[r * row_bytes + j] / divisor : 0.0f;
        }
        if (y) y[b] = ok ? (int64_t)(int8_t)labels[r] : -1;
    }
}
