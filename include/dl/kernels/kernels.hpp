#pragma once
// Every raw-pointer launcher of this build (the reference's kernels.hpp
// also listed elementwise, layernorm, transpose and vector_add, which are not
// on the GEMM path and are not provided).

#include <dl/kernels/activation.hpp>
#include <dl/kernels/bias.hpp>
#include <dl/kernels/cross_entropy.hpp>
#include <dl/kernels/gemm.hpp>
#include <dl/kernels/random.hpp>
#include <dl/kernels/reduction.hpp>
#include <dl/kernels/sgd.hpp>
#include <dl/kernels/softmax.hpp>
