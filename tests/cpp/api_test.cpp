// C++ dl:: API checks on the GPU, in the reference's test style: each check
// prints "<name> : passed|not passed" and the program exits non-zero if any
// fails.  Host loops here are the checker (same loops as the reference tests:
// matmul_tensor_test.cpp:9-25, linear_tensor_test.cpp:9-29).
#include <dl/dl.hpp>
#include <dl/kernels/kernels.hpp>

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <functional>
#include <iostream>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int g_failures = 0;

void report(const std::string& name, bool ok) {
    std::cout << name << " : " << (ok ? "passed" : "not passed") << std::endl;
    if (!ok) ++g_failures;
}

void run(const std::string& name, const std::function<bool()>& fn) {
    bool ok = false;
    try {
        ok = fn();
    } catch (const std::exception& e) {
        std::cout << name << " threw: " << e.what() << std::endl;
        ok = false;
    }
    report(name, ok);
}

std::string message_of(const std::function<void()>& fn) {
    try {
        fn();
    } catch (const std::exception& e) {
        return e.what();
    }
    return "";
}

std::vector<float> host_gemm(const std::vector<float>& a, const std::vector<float>& b, int m,
                             int n, int k, bool ta = false, bool tb = false) {
    std::vector<float> c(static_cast<std::size_t>(m) * n);
    for (int i = 0; i < m; ++i)
        for (int j = 0; j < n; ++j) {
            double s = 0;
            for (int kk = 0; kk < k; ++kk) {
                const float x = ta ? a[kk * m + i] : a[i * k + kk];
                const float y = tb ? b[j * k + kk] : b[kk * n + j];
                s += static_cast<double>(x) * y;
            }
            c[static_cast<std::size_t>(i) * n + j] = static_cast<float>(s);
        }
    return c;
}

bool close(const std::vector<float>& x, const std::vector<float>& y, float rel) {
    if (x.size() != y.size()) return false;
    float scale = 0;
    for (float v : y) scale = std::max(scale, std::fabs(v));
    for (std::size_t i = 0; i < x.size(); ++i) {
        if (!(std::fabs(x[i] - y[i]) <= rel * std::max(1.0f, scale))) return false;
    }
    return true;
}

std::vector<float> randv(std::size_t n, uint32_t seed, float lo = -1, float hi = 1) {
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = d(gen);
    return v;
}

const dl::Device kDev(dl::DeviceType::CUDA, 0);

}  // namespace

// Exported by libfastdl.so for tests (fast_dl_amd/csrc/dl/tensor/block_cache.hpp).
namespace dl {
namespace detail {
void inject_alloc_failures(int n);
}
}  // namespace dl

namespace {

}  // namespace

int main() {
    run("matmul_fixture", [] {
        // tests/tensor/matmul_tensor_test.cpp:30-42
        auto a = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6}, dl::Shape({2, 3}), kDev);
        auto b = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12},
                                              dl::Shape({3, 4}), kDev);
        auto c = dl::ops::matmul(a, b);
        const std::vector<float> want = {38, 44, 50, 56, 83, 98, 113, 128};
        return c.shape().rank() == 2 && c.shape()[0] == 2 && c.shape()[1] == 4 &&
               c.to_host<float>() == want;
    });

    run("linear_fixture", [] {
        // tests/tensor/linear_tensor_test.cpp:38-53
        auto x = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6}, dl::Shape({2, 3}), kDev);
        auto w = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6}, dl::Shape({3, 2}), kDev);
        auto b = dl::Tensor::from_host<float>({0.5f, 1.0f}, dl::Shape({2}), kDev);
        auto y = dl::ops::linear(x, w, b).to_host<float>();
        const std::vector<float> want = {22.5f, 29.0f, 49.5f, 65.0f};
        for (int i = 0; i < 4; ++i)
            if (std::fabs(y[i] - want[i]) > 1e-4f) return false;
        auto yr = dl::ops::linear_relu(x, w, dl::Tensor::from_host<float>({-100.f, 1.f},
                                                                           dl::Shape({2}), kDev))
                      .to_host<float>();
        return yr[0] == 0.0f && yr[2] == 0.0f && std::fabs(yr[1] - 29.0f) < 1e-4f;
    });

    run("matmul_skinny_k_split", [] {
        // 3 x 4096 times 4096 x 1024: the skinny family's K-split form, its
        // partials in a workspace from the block cache.  Repeated calls on the
        // null stream and on a user stream (each reusing the cached
        // workspace) give the same bits.
        const int m = 3, k = 4096, n = 1024;
        auto a = randv(m * k, 21), b = randv(k * n, 22);
        auto want = host_gemm(a, b, m, n, k);
        auto ta = dl::Tensor::from_host<float>(a, dl::Shape({m, k}), kDev);
        auto tb = dl::Tensor::from_host<float>(b, dl::Shape({k, n}), kDev);
        const auto first = dl::ops::matmul(ta, tb).to_host<float>();
        bool ok = close(first, want, 1e-5f) && dl::ops::matmul(ta, tb).to_host<float>() == first;
        dl::Stream s(kDev);
        {
            dl::StreamGuard g(s);
            auto c1 = dl::ops::matmul(ta, tb);
            auto c2 = dl::ops::matmul(ta, tb);
            dl::synchronize();
            ok = ok && c1.to_host<float>() == first && c2.to_host<float>() == first;
        }
        return ok;
    });

    run("matmul_random_all_algos", [] {
        const int m = 100, n = 70, k = 50;
        auto a = randv(m * k, 1), b = randv(k * n, 2);
        auto want = host_gemm(a, b, m, n, k);
        auto ta = dl::Tensor::from_host<float>(a, dl::Shape({m, k}), kDev);
        auto tb = dl::Tensor::from_host<float>(b, dl::Shape({k, n}), kDev);
        if (!close(dl::ops::matmul(ta, tb).to_host<float>(), want, 1e-5f)) return false;
        // The reference's four names (gemm_benchmark.cu:87-99 runs each) and this build's.
        for (auto algo : {dl::kernels::GemmAlgo::Naive, dl::kernels::GemmAlgo::Tiled,
                          dl::kernels::GemmAlgo::Register, dl::kernels::GemmAlgo::Cublas,
                          dl::kernels::GemmAlgo::Auto, dl::kernels::GemmAlgo::MfmaTiled128,
                          dl::kernels::GemmAlgo::MfmaTiled64, dl::kernels::GemmAlgo::MfmaSplitK}) {
            dl::Tensor tc(dl::Shape({m, n}), dl::DType::Float32, kDev);
            dl::kernels::gemm(static_cast<const float*>(ta.data()),
                              static_cast<const float*>(tb.data()), static_cast<float*>(tc.data()),
                              m, n, k, algo);
            if (!close(tc.to_host<float>(), want, 1e-5f)) {
                std::cout << "  algo " << dl::kernels::to_string(algo) << " mismatch" << std::endl;
                return false;
            }
        }
        return true;
    });

    run("matmul_direct_to_lds_algos", [] {
        // k and n multiples of 4: the direct-to-LDS kernels accept the shape;
        // k = 100 leaves a partial last K-tile for all three tiles.
        const int m = 300, n = 136, k = 100;
        auto a = randv(m * k, 11), b = randv(k * n, 12);
        auto want = host_gemm(a, b, m, n, k);
        auto ta = dl::Tensor::from_host<float>(a, dl::Shape({m, k}), kDev);
        auto tb = dl::Tensor::from_host<float>(b, dl::Shape({k, n}), kDev);
        for (auto algo : {dl::kernels::GemmAlgo::MfmaDma256, dl::kernels::GemmAlgo::MfmaDma128,
                          dl::kernels::GemmAlgo::MfmaDma64, dl::kernels::GemmAlgo::MfmaDma128W8,
                          dl::kernels::GemmAlgo::MfmaDma64U, dl::kernels::GemmAlgo::MfmaDma128W8U,
                          dl::kernels::GemmAlgo::MfmaDma64S, dl::kernels::GemmAlgo::MfmaDma96x32U}) {
            dl::Tensor tc(dl::Shape({m, n}), dl::DType::Float32, kDev);
            dl::kernels::gemm(static_cast<const float*>(ta.data()),
                              static_cast<const float*>(tb.data()), static_cast<float*>(tc.data()),
                              m, n, k, algo);
            if (!close(tc.to_host<float>(), want, 1e-5f)) {
                std::cout << "  algo " << dl::kernels::to_string(algo) << " mismatch" << std::endl;
                return false;
            }
        }
        // k % 4 != 0: a forced direct-to-LDS kernel is refused with an exception.
        const int k2 = 50;
        auto a2 = dl::Tensor::from_host<float>(randv(m * k2, 13), dl::Shape({m, k2}), kDev);
        auto b2 = dl::Tensor::from_host<float>(randv(k2 * n, 14), dl::Shape({k2, n}), kDev);
        dl::Tensor c2(dl::Shape({m, n}), dl::DType::Float32, kDev);
        try {
            dl::kernels::gemm(static_cast<const float*>(a2.data()),
                              static_cast<const float*>(b2.data()), static_cast<float*>(c2.data()),
                              m, n, k2, dl::kernels::GemmAlgo::MfmaDma128);
        } catch (const std::runtime_error&) {
            // ... while the 4-byte-copy twins take it.
            const auto want2 = host_gemm(a2.to_host<float>(), b2.to_host<float>(), m, n, k2);
            for (auto algo : {dl::kernels::GemmAlgo::MfmaDma64U,
                              dl::kernels::GemmAlgo::MfmaDma128W8U,
                              dl::kernels::GemmAlgo::MfmaDma96x32U}) {
                dl::kernels::gemm(static_cast<const float*>(a2.data()),
                                  static_cast<const float*>(b2.data()),
                                  static_cast<float*>(c2.data()), m, n, k2, algo);
                if (!close(c2.to_host<float>(), want2, 1e-5f)) {
                    std::cout << "  algo " << dl::kernels::to_string(algo) << " mismatch (k=50)"
                              << std::endl;
                    return false;
                }
            }
            return true;
        }
        std::cout << "  k % 4 != 0 was not refused" << std::endl;
        return false;
    });

    run("linear_backward", [] {
        const int rows = 33, in = 20, out = 7;
        auto x = randv(rows * in, 3), w = randv(in * out, 4), g = randv(rows * out, 5);
        auto tx = dl::Tensor::from_host<float>(x, dl::Shape({rows, in}), kDev);
        auto tw = dl::Tensor::from_host<float>(w, dl::Shape({in, out}), kDev);
        auto tg = dl::Tensor::from_host<float>(g, dl::Shape({rows, out}), kDev);
        auto grads = dl::ops::linear_backward(tg, tx, tw);
        // dX = dY W^T, dW = X^T dY, db = colsum(dY) (legacy/src/ops/Layers.cpp:36-44)
        auto dx = host_gemm(g, w, rows, in, out, false, true);
        auto dw = host_gemm(x, g, in, out, rows, true, false);
        std::vector<float> db(out, 0.0f);
        for (int r = 0; r < rows; ++r)
            for (int c = 0; c < out; ++c) db[c] += g[r * out + c];
        return close(grads.grad_input.to_host<float>(), dx, 1e-5f) &&
               close(grads.grad_weight.to_host<float>(), dw, 1e-5f) &&
               close(grads.grad_bias.to_host<float>(), db, 1e-5f) &&
               grads.grad_weight.shape()[0] == in && grads.grad_weight.shape()[1] == out;
    });

    run("relu_and_backward", [] {
        // tests/nn/relu_module_test.cpp:22-29
        auto x = dl::Tensor::from_host<float>({-2.f, -0.5f, 0.f, 1.5f, 3.f, -4.f},
                                              dl::Shape({2, 3}), kDev);
        dl::nn::ReLU relu;
        auto y = relu(x).to_host<float>();
        const std::vector<float> want = {0, 0, 0, 1.5f, 3.f, 0};
        auto g = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6}, dl::Shape({2, 3}), kDev);
        auto gi = dl::ops::relu_backward(g, x).to_host<float>();
        const std::vector<float> want_g = {0, 0, 0, 4, 5, 0};
        return y == want && gi == want_g && relu.parameters().empty();
    });

    run("cross_entropy_and_backward", [] {
        // tests/tensor/cross_entropy_tensor_test.cpp:40-44 -> 0.4076059
        auto z = dl::Tensor::from_host<float>({1, 2, 3, 1, 3, 2}, dl::Shape({2, 3}), kDev);
        auto lab = dl::Tensor::from_host<int64_t>({2, 1}, dl::Shape({2}), kDev);
        auto loss = dl::ops::cross_entropy(z, lab).to_host<float>();
        auto g = dl::ops::cross_entropy_backward(z, lab).to_host<float>();
        const double e = std::exp(1.0), s = 1 + e + e * e;
        // row 0: p = [1, e, e^2] / s, label 2
        const double want0[3] = {1 / s / 2, e / s / 2, (e * e / s - 1) / 2};
        bool ok = std::fabs(loss[0] - 0.4076059f) < 1e-4f;
        for (int c = 0; c < 3; ++c) ok = ok && std::fabs(g[c] - want0[c]) < 1e-6;
        return ok;
    });

    run("softmax_rows", [] {
        auto x = dl::Tensor::from_host<float>({1, 2, 3, 4, 1, 3, 2, 0}, dl::Shape({2, 4}), kDev);
        auto y = dl::ops::softmax(x).to_host<float>();
        float s0 = 0, s1 = 0;
        for (int c = 0; c < 4; ++c) {
            s0 += y[c];
            s1 += y[4 + c];
        }
        return std::fabs(s0 - 1) < 1e-5f && std::fabs(s1 - 1) < 1e-5f && y[3] > y[2];
    });

    run("error_messages", [] {
        // messages of src/ops/OpUtils.cpp and Matmul.cpp / Linear.cpp
        auto a = dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6}, dl::Shape({2, 3}), kDev);
        auto bad = dl::Tensor::from_host<float>({1, 2, 3, 4}, dl::Shape({2, 2}), kDev);
        auto i64 = dl::Tensor::from_host<int64_t>({1, 2}, dl::Shape({1, 2}), kDev);
        auto bias3 = dl::Tensor::from_host<float>({1, 2, 3}, dl::Shape({3}), kDev);
        dl::Tensor undefined;
        return message_of([&] { dl::ops::matmul(a, bad); }) ==
                   "matmul input tensors have incompatible shapes" &&
               message_of([&] { dl::ops::matmul(undefined, a); }) ==
                   "matmul: left tensor is not defined" &&
               message_of([&] { dl::ops::matmul(a, i64); }) == "matmul: right tensor must be float32" &&
               message_of([&] { dl::ops::matmul(bias3, a); }) ==
                   "matmul: left tensor has incorrect rank" &&
               message_of([&] { dl::ops::linear(a, bad, bias3); }) ==
                   "linear input and weight tensors have incompatible shapes" &&
               message_of([&] {
                   dl::ops::linear(a, dl::Tensor::from_host<float>({1, 2, 3, 4, 5, 6},
                                                                  dl::Shape({3, 2}), kDev),
                                   bias3);
               }) == "linear bias shape must be [out_features]";
    });

    run("sequential_mlp_forward", [] {
        dl::nn::Sequential model;
        model.add(std::make_unique<dl::nn::Linear>(5, 4, kDev));
        model.add(std::make_unique<dl::nn::ReLU>());
        model.add(std::make_unique<dl::nn::Linear>(4, 3, kDev));
        auto params = model.parameters();
        auto x = randv(2 * 5, 6);
        auto y = model(dl::Tensor::from_host<float>(x, dl::Shape({2, 5}), kDev)).to_host<float>();
        auto w1 = params[0]->to_host<float>(), b1 = params[1]->to_host<float>();
        auto w2 = params[2]->to_host<float>(), b2 = params[3]->to_host<float>();
        auto h = host_gemm(x, w1, 2, 4, 5);
        for (int r = 0; r < 2; ++r)
            for (int c = 0; c < 4; ++c) h[r * 4 + c] = std::max(0.0f, h[r * 4 + c] + b1[c]);
        auto want = host_gemm(h, w2, 2, 3, 4);
        for (int r = 0; r < 2; ++r)
            for (int c = 0; c < 3; ++c) want[r * 3 + c] += b2[c];
        // Kaiming-uniform range +-sqrt(6/in), zero bias (linear_kaiming_init_test.cpp:31-54)
        bool init_ok = true;
        for (float v : w1) init_ok = init_ok && std::fabs(v) <= std::sqrt(6.0f / 5) + 1e-6f;
        for (float v : b1) init_ok = init_ok && v == 0.0f;
        return params.size() == 4 && init_ok && close(y, want, 1e-5f);
    });

    run("sgd_and_mlp2_training", [] {
        const int batch = 64, in = 32, hidden = 16, classes = 10;
        dl::train::Mlp2 net(in, hidden, classes, batch, kDev, 99);
        auto x = dl::Tensor::from_host<float>(randv(batch * in, 7, 0, 1), dl::Shape({batch, in}), kDev);
        std::vector<int64_t> lab(batch);
        for (int i = 0; i < batch; ++i) lab[i] = (i * 7) % classes;
        auto labels = dl::Tensor::from_host<int64_t>(lab, dl::Shape({batch}), kDev);
        const float first = net.step(x, labels, 0.5f);
        float last = first;
        for (int s = 0; s < 30; ++s) last = net.step(x, labels, 0.5f);
        // SGD on its own: p - lr * g
        auto p = dl::Tensor::from_host<float>({1, 2, 3}, dl::Shape({3}), kDev);
        auto g = dl::Tensor::from_host<float>({1, 1, -2}, dl::Shape({3}), kDev);
        dl::optim::SGD opt(0.5f);
        opt.step({&p}, {&g});
        const std::vector<float> want = {0.5f, 1.5f, 4.0f};
        return std::isfinite(first) && last < first && p.to_host<float>() == want;
    });

    run("random_fills", [] {
        auto a = dl::Tensor::uniform(dl::Shape({1000}), dl::DType::Float32, kDev, -1, 2, 5).to_host<float>();
        auto b = dl::Tensor::uniform(dl::Shape({1000}), dl::DType::Float32, kDev, -1, 2, 5).to_host<float>();
        bool ok = a == b;
        for (float v : a) ok = ok && v > -1.0f && v <= 2.0f;
        auto n = dl::Tensor::randn(dl::Shape({4096}), dl::DType::Float32, kDev, 0, 1, 3).to_host<float>();
        double mean = 0;
        for (float v : n) mean += v;
        mean /= n.size();
        return ok && std::fabs(mean) < 0.1;
    });

    run("stream_guard_ops_match_null_stream", [] {
        // The same ops enqueued on a user stream give the same bits as on the
        // null stream (every kernel is deterministic), device copies and zero
        // fills follow the stream order, and the guard restores the stream.
        const int m = 300, k = 200, n = 170;
        auto a = dl::Tensor::from_host<float>(randv(m * k, 11), dl::Shape({m, k}), kDev);
        auto b = dl::Tensor::from_host<float>(randv(k * n, 12), dl::Shape({k, n}), kDev);
        auto bias = dl::Tensor::from_host<float>(randv(n, 13), dl::Shape({n}), kDev);
        const auto ref_mm = dl::ops::matmul(a, b).to_host<float>();
        const auto ref_lin = dl::ops::relu(dl::ops::linear(a, b, bias)).to_host<float>();
        bool ok = dl::current_stream() == nullptr;
        dl::Stream s(kDev);
        std::vector<float> mm, lin, copied, zeroed;
        {
            dl::StreamGuard g(s);
            ok = ok && dl::current_stream() == s.handle();
            auto c = dl::ops::matmul(a, b);
            auto y = dl::ops::relu(dl::ops::linear(a, b, bias));
            auto c2 = dl::Tensor::empty(c.shape(), dl::DType::Float32, kDev);
            c2.copy_from(c);
            auto z = dl::ops::matmul(a, b);
            z.zero_();
            dl::synchronize();
            mm = c.to_host<float>();
            lin = y.to_host<float>();
            copied = c2.to_host<float>();
            zeroed = z.to_host<float>();
        }
        ok = ok && dl::current_stream() == nullptr;
        bool zeros = true;
        for (float v : zeroed) zeros = zeros && v == 0.0f;
        return ok && mm == ref_mm && lin == ref_lin && copied == ref_mm && zeros;
    });

    // Tensor::zeros inside a captured graph: zero_ is a kernel, not a memset
    // node, so every replay zeroes the bias again (the bias and C are dirtied
    // with NaN between replays by eager work on the same stream).
    run("zeros_captured_in_a_graph_replays", [] {
        const int m = 64, n = 48, k = 32;
        const auto a = randv(static_cast<std::size_t>(m) * k, 41);
        const auto b = randv(static_cast<std::size_t>(k) * n, 42);
        const auto want = host_gemm(a, b, m, n, k);
        dl::Stream s(kDev);
        dl::StreamGuard guard(s);
        const hipStream_t hs = static_cast<hipStream_t>(s.handle());
        auto ta = dl::Tensor::from_host<float>(a, dl::Shape({m, k}), kDev);
        auto tb = dl::Tensor::from_host<float>(b, dl::Shape({k, n}), kDev);
        dl::Tensor c(dl::Shape({m, n}), dl::DType::Float32, kDev);
        // a cached block of the bias's size on this stream: the capture allocates nothing
        { dl::Tensor warm = dl::Tensor::zeros(dl::Shape({n}), dl::DType::Float32, kDev); }
        s.synchronize();
        dl::Tensor bias;
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        bool ok = hipStreamBeginCapture(hs, hipStreamCaptureModeThreadLocal) == hipSuccess;
        bias = dl::Tensor::zeros(dl::Shape({n}), dl::DType::Float32, kDev);
        dl::kernels::gemm_ex(dl::kernels::Transpose::No, dl::kernels::Transpose::No, m, n, k,
                             static_cast<const float*>(ta.data()), k, 0,
                             static_cast<const float*>(tb.data()), n, 0,
                             static_cast<float*>(c.data()), n, 0, 1,
                             static_cast<const float*>(bias.data()), nullptr,
                             dl::kernels::Epilogue::Bias, dl::kernels::GemmAlgo::Auto, hs);
        ok = hipStreamEndCapture(hs, &graph) == hipSuccess && ok;
        ok = ok && hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
        const std::vector<float> nan_bias(n, std::nanf("")), nan_c(m * n, std::nanf(""));
        for (int rep = 0; rep < 4 && ok; ++rep) {
            bias.copy_from_host(nan_bias.data(), nan_bias.size() * sizeof(float));
            c.copy_from_host(nan_c.data(), nan_c.size() * sizeof(float));
            ok = hipGraphLaunch(exec, hs) == hipSuccess && hipStreamSynchronize(hs) == hipSuccess;
            ok = ok && close(c.to_host<float>(), want, 1e-5f);
            std::vector<float> zeros = bias.to_host<float>();
            for (float v : zeros) ok = ok && v == 0.0f;
        }
        if (exec) ok = hipGraphExecDestroy(exec) == hipSuccess && ok;
        if (graph) ok = hipGraphDestroy(graph) == hipSuccess && ok;
        return ok;
    });

    run("mlp2_graph_replays_match_eager_steps_on_a_stream", [] {
        const int batch = 64, in = 32, hidden = 16, classes = 10;
        dl::train::Mlp2 eager(in, hidden, classes, batch, kDev, 5);
        dl::train::Mlp2 graphed(in, hidden, classes, batch, kDev, 5);
        auto x = dl::Tensor::from_host<float>(randv(batch * in, 21, 0, 1), dl::Shape({batch, in}), kDev);
        std::vector<int64_t> lab(batch);
        for (int i = 0; i < batch; ++i) lab[i] = (i * 3 + 1) % classes;
        auto labels = dl::Tensor::from_host<int64_t>(lab, dl::Shape({batch}), kDev);
        bool threw = false;
        try {
            graphed.replay();
        } catch (const std::runtime_error&) {
            threw = true;
        }
        dl::Stream s(kDev);
        dl::StreamGuard g(s);
        graphed.capture(x, labels, 0.25f);
        bool ok = threw;
        for (int i = 0; i < 4; ++i) {
            const float le = eager.step(x, labels, 0.25f);
            const float lg = graphed.replay();
            ok = ok && std::isfinite(le) && le == lg;
        }
        ok = ok && eager.w1().to_host<float>() == graphed.w1().to_host<float>() &&
             eager.b1().to_host<float>() == graphed.b1().to_host<float>() &&
             eager.w2().to_host<float>() == graphed.w2().to_host<float>() &&
             eager.b2().to_host<float>() == graphed.b2().to_host<float>();
        return ok;
    });

    run("mlp2_multi_step_graph_matches_eager_steps", [] {
        // A graph of three steps replayed twice: six eager steps' parameters
        // and last loss, bit for bit; steps < 1 is refused.
        const int batch = 64, in = 32, hidden = 16, classes = 10;
        dl::train::Mlp2 eager(in, hidden, classes, batch, kDev, 7);
        dl::train::Mlp2 graphed(in, hidden, classes, batch, kDev, 7);
        auto x = dl::Tensor::from_host<float>(randv(batch * in, 23, 0, 1), dl::Shape({batch, in}), kDev);
        std::vector<int64_t> lab(batch);
        for (int i = 0; i < batch; ++i) lab[i] = (i * 7 + 2) % classes;
        auto labels = dl::Tensor::from_host<int64_t>(lab, dl::Shape({batch}), kDev);
        bool threw = false;
        try {
            graphed.capture(x, labels, 0.25f, 0);
        } catch (const std::runtime_error&) {
            threw = true;
        }
        dl::Stream s(kDev);
        dl::StreamGuard g(s);
        graphed.capture(x, labels, 0.25f, 3);
        bool ok = threw;
        for (int rep = 0; rep < 2; ++rep) {
            float le = 0.0f;
            for (int i = 0; i < 3; ++i) le = eager.step(x, labels, 0.25f);
            const float lg = graphed.replay();
            ok = ok && std::isfinite(le) && le == lg;
        }
        ok = ok && eager.w1().to_host<float>() == graphed.w1().to_host<float>() &&
             eager.b1().to_host<float>() == graphed.b1().to_host<float>() &&
             eager.w2().to_host<float>() == graphed.w2().to_host<float>() &&
             eager.b2().to_host<float>() == graphed.b2().to_host<float>();
        return ok;
    });

    // The block cache: a tensor allocated on stream T and freed while S is
    // current goes back to T, so S cannot overwrite it under T's queued work.
    run("allocator_freed_block_returns_to_home_stream", [] {
        const int n = 1024;
        const auto hx = randv(static_cast<std::size_t>(n) * n, 31);
        const auto hw = randv(static_cast<std::size_t>(n) * 16, 32);
        dl::Stream t(kDev), s(kDev);
        auto w = dl::Tensor::from_host<float>(hw, dl::Shape({n, 16}), kDev);
        auto big = dl::Tensor::from_host<float>(randv(4096 * 4096, 33), dl::Shape({4096, 4096}), kDev);
        dl::Tensor c, y, busy;
        const void* xp = nullptr;
        bool ok = true;
        {
            std::vector<dl::Tensor> holder;
            {
                dl::StreamGuard g(t);
                holder.push_back(dl::Tensor::from_host<float>(hx, dl::Shape({n, n}), kDev));
                xp = holder[0].data();
                busy = dl::ops::matmul(big, big);     // about 1 ms of work queued first
                c = dl::ops::matmul(holder[0], w);    // then the product that reads x
            }
            dl::StreamGuard g(s);
            holder.clear();                            // x dies while S is current
            y = dl::Tensor(dl::Shape({n, n}), dl::DType::Float32, kDev);
            ok = ok && y.data() != xp;
            y.zero_();                                 // S writes its new block at once
        }
        t.synchronize();
        s.synchronize();
        ok = ok && close(c.to_host<float>(), host_gemm(hx, hw, n, 16, n), 1e-4f);
        dl::StreamGuard g(t);
        dl::Tensor z(dl::Shape({n, n}), dl::DType::Float32, kDev);
        return ok && z.data() == xp;
    });

    // Allocated on S, read by a product queued on T: when it dies under S the
    // block waits for T to pass that point before S can have it again.
    run("allocator_block_used_on_another_stream_waits", [] {
        const int n = 1024;
        const auto hx = randv(static_cast<std::size_t>(n) * n, 41);
        const auto hw = randv(static_cast<std::size_t>(n) * 16, 42);
        dl::Stream t(kDev), s(kDev);
        auto w = dl::Tensor::from_host<float>(hw, dl::Shape({n, 16}), kDev);
        auto big = dl::Tensor::from_host<float>(randv(4096 * 4096, 43), dl::Shape({4096, 4096}), kDev);
        dl::Tensor c, busy;
        const void* xp = nullptr;
        {
            dl::StreamGuard gs(s);
            std::vector<dl::Tensor> holder;
            holder.push_back(dl::Tensor::from_host<float>(hx, dl::Shape({n, n}), kDev));
            xp = holder[0].data();
            {
                dl::StreamGuard gt(t);
                busy = dl::ops::matmul(big, big);
                c = dl::ops::matmul(holder[0], w);  // records T as a user of x
            }
            holder.clear();
            dl::Tensor y(dl::Shape({n, n}), dl::DType::Float32, kDev);
            y.zero_();
        }
        t.synchronize();
        s.synchronize();
        bool ok = close(c.to_host<float>(), host_gemm(hx, hw, n, 16, n), 1e-4f);
        dl::StreamGuard gs(s);
        dl::Tensor again(dl::Shape({n, n}), dl::DType::Float32, kDev);  // T passed: reusable
        return ok && again.data() == xp;
    });

    // An allocation that fails for real (the test hook asks the runtime for an
    // impossible size once) is retried after the cache is emptied, and the
    // failure does not surface in the next op.
    run("allocator_out_of_memory_retry_leaves_no_error", [] {
        const int m = 64, k = 48, n = 32;
        const auto ha = randv(m * k, 51), hb = randv(k * n, 52);
        { dl::Tensor warm(dl::Shape({4096}), dl::DType::Float32, kDev); }  // a cached block to free
        dl::detail::inject_alloc_failures(1);
        auto a = dl::Tensor::from_host<float>(ha, dl::Shape({m, k}), kDev);
        auto b = dl::Tensor::from_host<float>(hb, dl::Shape({k, n}), kDev);
        auto c = dl::ops::matmul(a, b);
        return close(c.to_host<float>(), host_gemm(ha, hb, m, n, k), 1e-4f);
    });

    std::cout << "api_test : " << (g_failures == 0 ? "passed" : "not passed") << std::endl;
    return g_failures == 0 ? 0 : 1;
}
