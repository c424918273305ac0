#pragma once
// Mean softmax cross-entropy (reference include/dl/ops/CrossEntropy.hpp) and
// its gradient with respect to the logits.

#include <dl/tensor/Tensor.hpp>

namespace dl::ops {

// loss [1] = mean over the batch of logsumexp(z) - z[label]; labels int64.
Tensor cross_entropy(const Tensor& logits, const Tensor& labels);

// (softmax(z) - onehot(label)) / batch, shaped like logits
// (legacy/src/ops/SoftmaxCrossEntropyLoss.cpp:39-51).
Tensor cross_entropy_backward(const Tensor& logits, const Tensor& labels);

}  // namespace dl::ops
