#pragma once
// All ops of this build (the reference's Ops.hpp also pulled in elementwise
// and layernorm, which are not on the GEMM path and are not provided).

#include <dl/ops/Activation.hpp>
#include <dl/ops/CrossEntropy.hpp>
#include <dl/ops/Linear.hpp>
#include <dl/ops/Matmul.hpp>
#include <dl/ops/Softmax.hpp>
