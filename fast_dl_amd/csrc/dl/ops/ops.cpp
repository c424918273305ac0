// dl::ops on the gfx950 kernels.  Validation order and messages follow the
// reference (src/ops/OpUtils.cpp:20-101, Matmul.cpp:14-45, Linear.cpp:14-47,
// Activation.cpp:13-34, Softmax.cpp:14-42, CrossEntropy.cpp:14-43); the
// compute differs: linear's bias is fused into the GEMM epilogue instead of a
// second pass over the output.  matmul, linear, linear_relu, relu and
// cross_entropy record their backward node when an input requires a gradient.
#include "../autograd/record.hpp"
#include "../kernels/sgemm_call.hpp"

#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/kernels/kernels.hpp>
#include <dl/ops/Ops.hpp>
#include <dl/ops/OpUtils.hpp>

#include <fastdl_gemm.h>

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace dl::ops {

namespace {

std::string prefix(const char* op) { return std::string(op) + ": "; }

void set_device(const Tensor& t) {
    hip::check(hipSetDevice(t.device().index), "cudaSetDevice failed");
}

const float* f32(const Tensor& t) { return static_cast<const float*>(t.data()); }
float* f32(Tensor& t) { return static_cast<float*>(t.data()); }

}  // namespace

// ------------------------------------------------------------------ OpUtils

void check_defined(const Tensor& t, const char* op, const char* name) {
    if (!t.defined()) throw std::runtime_error(prefix(op) + name + " tensor is not defined");
}

void check_rank(const Tensor& t, int64_t rank, const char* op, const char* name) {
    if (t.shape().rank() != rank) throw std::runtime_error(prefix(op) + name + " tensor has incorrect rank");
}

void check_cuda(const Tensor& t, const char* op, const char* name) {
    if (!t.device().is_cuda()) throw std::runtime_error(prefix(op) + name + " tensor must be CUDA");
}

void check_dtype(const Tensor& t, DType dtype, const char* op, const char* name) {
    if (t.dtype() != dtype) {
        throw std::runtime_error(prefix(op) + name + " tensor must be " + dtype_name(dtype));
    }
}

void check_float32(const Tensor& t, const char* op, const char* name) {
    check_dtype(t, DType::Float32, op, name);
}

void check_same_device(const Tensor& a, const Tensor& b, const char* op, const char* an,
                       const char* bn) {
    if (a.device().type != b.device().type || a.device().index != b.device().index) {
        throw std::runtime_error(prefix(op) + an + " and " + bn + " tensors must be on the same device");
    }
}

void check_same_dtype(const Tensor& a, const Tensor& b, const char* op, const char* an,
                      const char* bn) {
    if (a.dtype() != b.dtype()) {
        throw std::runtime_error(prefix(op) + an + " and " + bn + " tensors must have the same dtype");
    }
}

void check_same_shape(const Tensor& a, const Tensor& b, const char* op, const char* an,
                      const char* bn) {
    if (a.shape().dims != b.shape().dims) {
        throw std::runtime_error(prefix(op) + an + " and " + bn + " tensors must have the same shape");
    }
}

void check_binary_float_cuda_op(const Tensor& a, const Tensor& b, const char* op) {
    check_defined(a, op, "left");
    check_defined(b, op, "right");
    check_same_shape(a, b, op);
    check_same_dtype(a, b, op);
    check_float32(a, op, "left");
    check_cuda(a, op, "left");
    check_cuda(b, op, "right");
    check_same_device(a, b, op);
}

// ------------------------------------------------------------------- matmul

Tensor matmul(const Tensor& a, const Tensor& b) {
    check_defined(a, "matmul", "left");
    check_defined(b, "matmul", "right");
    check_rank(a, 2, "matmul", "left");
    check_rank(b, 2, "matmul", "right");
    check_float32(a, "matmul", "left");
    check_float32(b, "matmul", "right");
    check_cuda(a, "matmul", "left");
    check_cuda(b, "matmul", "right");
    check_same_device(a, b, "matmul");
    if (a.shape()[1] != b.shape()[0]) {
        throw std::runtime_error("matmul input tensors have incompatible shapes");
    }
    const int64_t m = a.shape()[0], k = a.shape()[1], n = b.shape()[1];
    Tensor out(Shape({m, n}), a.dtype(), a.device());
    set_device(a);
    hip::check_fdl(detail::sgemm_auto(FDL_OP_N, FDL_OP_N, m, n, k, f32(a), k, 0, f32(b), n, 0,
                                f32(out), n, 0, 1, nullptr, nullptr, FDL_EPILOGUE_NONE, current_stream()),
                   "matmul kernel launch failed");
    if (autograd::any_requires_grad({&a, &b})) {
        autograd::record(out, autograd::make_matmul_backward(a, b));
    }
    return out;
}

// ------------------------------------------------------------------- linear

namespace {

void check_linear(const Tensor& input, const Tensor& weight, const Tensor& bias, const char* op) {
    check_defined(input, op, "input");
    check_defined(weight, op, "weight");
    check_defined(bias, op, "bias");
    check_rank(input, 2, op, "input");
    check_rank(weight, 2, op, "weight");
    check_rank(bias, 1, op, "bias");
    check_float32(input, op, "input");
    check_same_dtype(input, weight, op, "input", "weight");
    check_same_dtype(input, bias, op, "input", "bias");
    check_cuda(input, op, "input");
    check_cuda(weight, op, "weight");
    check_cuda(bias, op, "bias");
    check_same_device(input, weight, op, "input", "weight");
    check_same_device(input, bias, op, "input", "bias");
    if (input.shape()[1] != weight.shape()[0]) {
        throw std::runtime_error("linear input and weight tensors have incompatible shapes");
    }
    if (weight.shape()[1] != bias.shape()[0]) {
        throw std::runtime_error("linear bias shape must be [out_features]");
    }
}

Tensor linear_impl(const Tensor& input, const Tensor& weight, const Tensor& bias, int epilogue,
                   const char* op) {
    check_linear(input, weight, bias, op);
    const int64_t rows = input.shape()[0], in = input.shape()[1], out_f = weight.shape()[1];
    Tensor out(Shape({rows, out_f}), input.dtype(), input.device());
    set_device(input);
    hip::check_fdl(detail::sgemm_auto(FDL_OP_N, FDL_OP_N, rows, out_f, in, f32(input), in, 0,
                                f32(weight), out_f, 0, f32(out), out_f, 0, 1, f32(bias), nullptr,
                                epilogue, current_stream()),
                   "linear kernel launch failed");
    return out;
}

}  // namespace

Tensor linear(const Tensor& input, const Tensor& weight, const Tensor& bias) {
    Tensor out = linear_impl(input, weight, bias, FDL_EPILOGUE_BIAS, "linear");
    if (autograd::any_requires_grad({&input, &weight, &bias})) {
        autograd::record(out, autograd::make_linear_backward(input, weight, bias));
    }
    return out;
}

Tensor linear_relu(const Tensor& input, const Tensor& weight, const Tensor& bias) {
    Tensor out = linear_impl(input, weight, bias, FDL_EPILOGUE_BIAS_RELU, "linear_relu");
    if (autograd::any_requires_grad({&input, &weight, &bias})) {
        autograd::record(out, autograd::make_linear_relu_backward(input, weight, bias, out));
    }
    return out;
}

LinearGrads linear_backward(const Tensor& grad_output, const Tensor& input, const Tensor& weight,
                            bool need_grad_input) {
    const char* op = "linear_backward";
    check_defined(grad_output, op, "grad_output");
    check_defined(input, op, "input");
    check_defined(weight, op, "weight");
    check_rank(grad_output, 2, op, "grad_output");
    check_rank(input, 2, op, "input");
    check_rank(weight, 2, op, "weight");
    check_float32(grad_output, op, "grad_output");
    check_float32(input, op, "input");
    check_float32(weight, op, "weight");
    check_cuda(grad_output, op, "grad_output");
    check_same_device(grad_output, input, op, "grad_output", "input");
    check_same_device(grad_output, weight, op, "grad_output", "weight");
    const int64_t rows = input.shape()[0], in = input.shape()[1], out_f = weight.shape()[1];
    if (weight.shape()[0] != in || grad_output.shape()[0] != rows ||
        grad_output.shape()[1] != out_f) {
        throw std::runtime_error("linear_backward tensors have incompatible shapes");
    }
    set_device(input);
    LinearGrads g;
    if (need_grad_input) {
        g.grad_input = Tensor(Shape({rows, in}), DType::Float32, input.device());
        // dX = dY W^T  (NT)
        hip::check_fdl(detail::sgemm_auto(FDL_OP_N, FDL_OP_T, rows, in, out_f, f32(grad_output), out_f, 0,
                                    f32(weight), out_f, 0, f32(g.grad_input), in, 0, 1, nullptr,
                                    nullptr, FDL_EPILOGUE_NONE, current_stream()),
                       "linear_backward grad_input failed");
    }
    // dW = X^T dY  (TN)
    g.grad_weight = Tensor(Shape({in, out_f}), DType::Float32, input.device());
    hip::check_fdl(detail::sgemm_auto(FDL_OP_T, FDL_OP_N, in, out_f, rows, f32(input), in, 0,
                                f32(grad_output), out_f, 0, f32(g.grad_weight), out_f, 0, 1,
                                nullptr, nullptr, FDL_EPILOGUE_NONE, current_stream()),
                   "linear_backward grad_weight failed");
    // db = column sums of dY
    g.grad_bias = Tensor(Shape({out_f}), DType::Float32, input.device());
    hip::check_fdl(fdl_colsum(f32(grad_output), f32(g.grad_bias), rows, out_f, current_stream()),
                   "linear_backward grad_bias failed");
    return g;
}

// -------------------------------------------------------------- activation

Tensor relu(const Tensor& input) {
    check_defined(input, "relu");
    check_float32(input, "relu");
    check_cuda(input, "relu");
    Tensor out(input.shape(), input.dtype(), input.device());
    set_device(input);
    hip::check_fdl(fdl_relu(f32(input), f32(out), input.numel(), current_stream()),
                   "activation kernel launch failed");
    if (input.requires_grad()) autograd::record(out, autograd::make_relu_backward(input));
    return out;
}

Tensor relu_backward(const Tensor& grad_output, const Tensor& activation) {
    check_binary_float_cuda_op(grad_output, activation, "relu_backward");
    Tensor out(grad_output.shape(), grad_output.dtype(), grad_output.device());
    set_device(grad_output);
    hip::check_fdl(fdl_relu_backward(f32(grad_output), f32(activation), f32(out),
                                     grad_output.numel(), current_stream()),
                   "relu_backward kernel launch failed");
    return out;
}

// ----------------------------------------------------------------- softmax

Tensor softmax(const Tensor& input) {
    check_defined(input, "softmax");
    check_rank(input, 2, "softmax");
    check_float32(input, "softmax");
    check_cuda(input, "softmax");
    const int64_t rows = input.shape()[0], cols = input.shape()[1];
    if (rows == 0 || cols == 0) throw std::runtime_error("softmax rows and cols must be non-zero");
    Tensor out(input.shape(), input.dtype(), input.device());
    set_device(input);
    hip::check_fdl(fdl_softmax(f32(input), f32(out), rows, cols, current_stream()),
                   "softmax kernel launch failed");
    return out;
}

// ----------------------------------------------------------- cross entropy

namespace {

void check_xent(const Tensor& logits, const Tensor& labels) {
    check_defined(logits, "cross_entropy", "logits");
    check_defined(labels, "cross_entropy", "labels");
    check_rank(logits, 2, "cross_entropy", "logits");
    check_rank(labels, 1, "cross_entropy", "labels");
    check_float32(logits, "cross_entropy", "logits");
    check_dtype(labels, DType::Int64, "cross_entropy", "labels");
    check_cuda(logits, "cross_entropy", "logits");
    check_cuda(labels, "cross_entropy", "labels");
    check_same_device(logits, labels, "cross_entropy", "logits", "labels");
    if (logits.shape()[0] != labels.shape()[0]) {
        throw std::runtime_error("cross_entropy logits and labels batch size mismatch");
    }
    if (logits.shape()[1] <= 0) {
        throw std::runtime_error("cross_entropy class count must be positive");
    }
}

}  // namespace

Tensor cross_entropy(const Tensor& logits, const Tensor& labels) {
    check_xent(logits, labels);
    Tensor loss(Shape({1}), DType::Float32, logits.device());
    set_device(logits);
    hip::check_fdl(fdl_softmax_xent(f32(logits), static_cast<const int64_t*>(labels.data()),
                                    f32(loss), nullptr, logits.shape()[0], logits.shape()[1],
                                    current_stream()),
                   "cross_entropy kernel launch failed");
    if (logits.requires_grad()) {
        autograd::record(loss, autograd::make_cross_entropy_backward(logits, labels));
    }
    return loss;
}

Tensor cross_entropy_backward(const Tensor& logits, const Tensor& labels) {
    check_xent(logits, labels);
    Tensor grad(logits.shape(), DType::Float32, logits.device());
    set_device(logits);
    hip::check_fdl(fdl_softmax_xent(f32(logits), static_cast<const int64_t*>(labels.data()),
                                    nullptr, f32(grad), logits.shape()[0], logits.shape()[1],
                                    current_stream()),
                   "cross_entropy_backward kernel launch failed");
    return grad;
}

}  // namespace dl::ops
