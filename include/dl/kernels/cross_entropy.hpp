#pragma once
// Mean softmax cross-entropy (reference include/dl/kernels/cross_entropy.hpp).
// *loss is written (the reference op zeroed it and accumulated into it; the
// value is the same).

#include <cstdint>

namespace dl::kernels {

void cross_entropy(const float* logits, const int64_t* labels, float* loss, int batch,
                   int classes);

// grad = (softmax(logits) - onehot(labels)) / batch; loss may be null.
void cross_entropy_backward(const float* logits, const int64_t* labels, float* loss,
                            float* grad, int batch, int classes);

}  // namespace dl::kernels
