// Autograd checks on the GPU, in the reference's test style ("<name> :
// passed|not passed", non-zero exit on a failure).  The checkers are the
// path's own explicit backward ops run by hand in the same order (the
// autograd nodes call the same kernels, so gradients must match bit for
// bit), host fp64 products for the NT/TN orientation of matmul's node, and
// the fused two-layer trainer for a full SGD step.
#include <dl/dl.hpp>

#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <iostream>
#include <memory>
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

bool throws(const std::function<void()>& fn) {
    try {
        fn();
    } catch (const std::exception&) {
        return true;
    }
    return false;
}

std::vector<float> randv(std::size_t n, uint32_t seed, float lo = -1, float hi = 1) {
    std::mt19937 gen(seed);
    std::uniform_real_distribution<float> d(lo, hi);
    std::vector<float> v(n);
    for (auto& x : v) x = d(gen);
    return v;
}

std::vector<int64_t> labels_of(int n, int classes, uint32_t seed) {
    std::mt19937 gen(seed);
    std::uniform_int_distribution<int> d(0, classes - 1);
    std::vector<int64_t> v(n);
    for (auto& x : v) x = d(gen);
    return v;
}

bool same_bits(const Tensor& a, const Tensor& b) {
    if (!a.defined() || !b.defined() || a.shape().dims != b.shape().dims) return false;
    const std::vector<float> x = a.to_host<float>(), y = b.to_host<float>();
    return std::memcmp(x.data(), y.data(), x.size() * sizeof(float)) == 0;
}

bool close(const std::vector<float>& x, const std::vector<double>& y, double rel) {
    if (x.size() != y.size()) return false;
    double scale = 0;
    for (double v : y) scale = std::max(scale, std::fabs(v));
    for (std::size_t i = 0; i < x.size(); ++i) {
        if (!(std::fabs(x[i] - y[i]) <= rel * std::max(1e-30, scale))) return false;
    }
    return true;
}

const dl::Device kDev(dl::DeviceType::CUDA, 0);

}  // namespace

int main() {
    run("matmul_node_gives_nt_and_tn_products", [] {
        const int m = 37, k = 19, n = 11;
        Tensor a = Tensor::from_host(randv(m * k, 1), Shape({m, k}), kDev);
        Tensor b = Tensor::from_host(randv(k * n, 2), Shape({k, n}), kDev);
        a.set_requires_grad();
        b.set_requires_grad();
        const Tensor labels = Tensor::from_host(labels_of(m, n, 3), Shape({m}), kDev);
        const Tensor c = dl::ops::matmul(a, b);
        const Tensor loss = dl::ops::cross_entropy(c, labels);
        bool ok = c.grad_fn() && c.grad_fn()->name() == "MatmulBackward" &&
                  loss.grad_fn()->name() == "CrossEntropyBackward";
        loss.backward();
        // dC from the explicit op, then dA = dC B^T and dB = A^T dC in fp64
        const std::vector<float> dc = dl::ops::cross_entropy_backward(c, labels).to_host<float>();
        const std::vector<float> ah = a.to_host<float>(), bh = b.to_host<float>();
        std::vector<double> da(m * k, 0.0), db(k * n, 0.0);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < n; ++j)
                for (int kk = 0; kk < k; ++kk) {
                    da[i * k + kk] += double(dc[i * n + j]) * bh[kk * n + j];
                    db[kk * n + j] += double(ah[i * k + kk]) * dc[i * n + j];
                }
        ok = ok && close(a.grad().to_host<float>(), da, 1e-5) &&
             close(b.grad().to_host<float>(), db, 1e-5);
        return ok && a.grad().shape().dims == a.shape().dims && !c.grad().defined();
    });

    run("a_tensor_used_twice_gets_both_contributions", [] {
        // C = A A: dA = dC A^T + A^T dC, accumulated from the node's two inputs.
        const int m = 23, classes = m;
        Tensor a = Tensor::from_host(randv(m * m, 31), Shape({m, m}), kDev);
        a.set_requires_grad();
        const Tensor labels = Tensor::from_host(labels_of(m, classes, 32), Shape({m}), kDev);
        const Tensor c = dl::ops::matmul(a, a);
        dl::ops::cross_entropy(c, labels).backward();
        const std::vector<float> dc = dl::ops::cross_entropy_backward(c, labels).to_host<float>();
        const std::vector<float> ah = a.to_host<float>();
        std::vector<double> da(m * m, 0.0);
        for (int i = 0; i < m; ++i)
            for (int j = 0; j < m; ++j)
                for (int k = 0; k < m; ++k) {
                    da[i * m + k] += double(dc[i * m + j]) * ah[k * m + j];  // dC A^T
                    da[k * m + j] += double(ah[i * m + k]) * dc[i * m + j];  // A^T dC
                }
        return close(a.grad().to_host<float>(), da, 1e-5);
    });

    run("mlp_gradients_equal_the_explicit_backward_ops", [] {
        const int batch = 64, in = 96, hidden = 48, classes = 10;
        dl::nn::Sequential model;
        model.add(std::make_unique<dl::nn::Linear>(in, hidden, kDev));
        model.add(std::make_unique<dl::nn::ReLU>());
        model.add(std::make_unique<dl::nn::Linear>(hidden, classes, kDev));
        const std::vector<Tensor*> params = model.parameters();
        for (Tensor* p : params) p->set_requires_grad();
        const Tensor x = Tensor::from_host(randv(batch * in, 4, 0, 1), Shape({batch, in}), kDev);
        const Tensor y = Tensor::from_host(labels_of(batch, classes, 5), Shape({batch}), kDev);
        const Tensor loss = dl::ops::cross_entropy(model.forward(x), y);
        loss.backward();
        // The same backward by hand with the explicit ops.
        Tensor& w1 = *params[0];
        Tensor& b1 = *params[1];
        Tensor& w2 = *params[2];
        Tensor& b2 = *params[3];
        const Tensor z1 = dl::ops::linear(x, w1, b1);
        const Tensor h = dl::ops::relu(z1);
        const Tensor logits = dl::ops::linear(h, w2, b2);
        const Tensor g2 = dl::ops::cross_entropy_backward(logits, y);
        const dl::ops::LinearGrads l2 = dl::ops::linear_backward(g2, h, w2, true);
        const Tensor g1 = dl::ops::relu_backward(l2.grad_input, z1);
        const dl::ops::LinearGrads l1 = dl::ops::linear_backward(g1, x, w1, false);
        return same_bits(w2.grad(), l2.grad_weight) && same_bits(b2.grad(), l2.grad_bias) &&
               same_bits(w1.grad(), l1.grad_weight) && same_bits(b1.grad(), l1.grad_bias) &&
               !x.requires_grad() && !x.grad().defined();
    });

    run("linear_relu_node_uses_its_output_mask", [] {
        const int batch = 33, in = 40, out = 24, classes = out;
        Tensor w = Tensor::from_host(randv(in * out, 6), Shape({in, out}), kDev);
        Tensor b = Tensor::from_host(randv(out, 7), Shape({out}), kDev);
        w.set_requires_grad();
        b.set_requires_grad();
        const Tensor x = Tensor::from_host(randv(batch * in, 8), Shape({batch, in}), kDev);
        const Tensor y = Tensor::from_host(labels_of(batch, classes, 9), Shape({batch}), kDev);
        const Tensor h = dl::ops::linear_relu(x, w, b);
        const Tensor loss = dl::ops::cross_entropy(h, y);
        loss.backward();
        const Tensor g = dl::ops::relu_backward(dl::ops::cross_entropy_backward(h, y), h);
        const dl::ops::LinearGrads lg = dl::ops::linear_backward(g, x, w, false);
        return h.grad_fn()->name() == "LinearReluBackward" && same_bits(w.grad(), lg.grad_weight) &&
               same_bits(b.grad(), lg.grad_bias);
    });

    run("gradients_accumulate_zero_and_drive_sgd", [] {
        const int batch = 16, in = 8, classes = 5;
        Tensor w = Tensor::from_host(randv(in * classes, 10), Shape({in, classes}), kDev);
        Tensor b = Tensor::zeros(Shape({classes}), DType::Float32, kDev);
        w.set_requires_grad();
        b.set_requires_grad();
        const Tensor x = Tensor::from_host(randv(batch * in, 11), Shape({batch, in}), kDev);
        const Tensor y = Tensor::from_host(labels_of(batch, classes, 12), Shape({batch}), kDev);
        dl::ops::cross_entropy(dl::ops::linear(x, w, b), y).backward();
        const std::vector<float> once = w.grad().to_host<float>();
        dl::ops::cross_entropy(dl::ops::linear(x, w, b), y).backward();
        const std::vector<float> twice = w.grad().to_host<float>();
        bool ok = true;
        for (std::size_t i = 0; i < once.size(); ++i) ok = ok && twice[i] == 2.0f * once[i];
        dl::optim::SGD::zero_grad({&w, &b});
        ok = ok && !w.grad().defined() && !b.grad().defined();
        dl::ops::cross_entropy(dl::ops::linear(x, w, b), y).backward();
        const std::vector<float> w0 = w.to_host<float>(), g = w.grad().to_host<float>();
        dl::optim::SGD(0.5f).step({&w, &b});
        const std::vector<float> w1 = w.to_host<float>();
        for (std::size_t i = 0; i < w0.size(); ++i) {
            const float lg = 0.5f * g[i];
            ok = ok && w1[i] == w0[i] - lg;
        }
        return ok;
    });

    run("autograd_step_matches_the_fused_trainer", [] {
        const int batch = 128, in = 784, hidden = 256, classes = 10;
        dl::train::Mlp2 fused(in, hidden, classes, batch, kDev, 21);
        Tensor w1 = Tensor::empty(fused.w1().shape(), DType::Float32, kDev);
        Tensor b1 = Tensor::empty(fused.b1().shape(), DType::Float32, kDev);
        Tensor w2 = Tensor::empty(fused.w2().shape(), DType::Float32, kDev);
        Tensor b2 = Tensor::empty(fused.b2().shape(), DType::Float32, kDev);
        w1.copy_from(fused.w1());
        b1.copy_from(fused.b1());
        w2.copy_from(fused.w2());
        b2.copy_from(fused.b2());
        for (Tensor* p : {&w1, &b1, &w2, &b2}) p->set_requires_grad();
        const Tensor x = Tensor::from_host(randv(batch * in, 22, 0, 1), Shape({batch, in}), kDev);
        const Tensor y = Tensor::from_host(labels_of(batch, classes, 23), Shape({batch}), kDev);
        const float lr = 0.1f;
        bool ok = true;
        for (int step = 0; step < 3; ++step) {
            const Tensor loss = dl::ops::cross_entropy(
                dl::ops::linear(dl::ops::linear_relu(x, w1, b1), w2, b2), y);
            loss.backward();
            dl::optim::SGD(lr).step({&w1, &b1, &w2, &b2});
            dl::optim::SGD::zero_grad({&w1, &b1, &w2, &b2});
            const float fused_loss = fused.step(x, y, lr);
            const float auto_loss = loss.to_host<float>()[0];
            ok = ok && std::fabs(fused_loss - auto_loss) <= 1e-5f * std::fabs(fused_loss);
        }
        // different summation orders (the fused head's per-block records):
        // the parameters agree to a few ulps of their scale
        const auto rel = [](const Tensor& a, const Tensor& b) {
            const std::vector<float> x = a.to_host<float>(), y = b.to_host<float>();
            double num = 0, den = 0;
            for (std::size_t i = 0; i < x.size(); ++i) {
                num = std::max(num, std::fabs(double(x[i]) - y[i]));
                den = std::max(den, std::fabs(double(y[i])));
            }
            return num / std::max(den, 1e-30);
        };
        return ok && rel(w1, fused.w1()) < 2e-5 && rel(b1, fused.b1()) < 2e-5 &&
               rel(w2, fused.w2()) < 2e-5 && rel(b2, fused.b2()) < 2e-5;
    });

    run("no_graph_without_requires_grad_and_argument_checks", [] {
        const Tensor a = Tensor::from_host(randv(12, 13), Shape({3, 4}), kDev);
        const Tensor b = Tensor::from_host(randv(8, 14), Shape({4, 2}), kDev);
        const Tensor c = dl::ops::matmul(a, b);
        bool ok = !c.grad_fn() && !c.requires_grad();
        const Tensor labels = Tensor::from_host(std::vector<int64_t>{0, 1, 1}, Shape({3}), kDev);
        const Tensor loss = dl::ops::cross_entropy(c, labels);
        ok = ok && throws([&] { loss.backward(); });  // nothing requires a gradient
        Tensor w = Tensor::from_host(randv(8, 15), Shape({4, 2}), kDev);
        w.set_requires_grad();
        const Tensor c2 = dl::ops::matmul(a, w);
        ok = ok && throws([&] { c2.backward(); });            // more than one element
        Tensor c2m = c2;
        ok = ok && throws([&] { c2m.set_requires_grad(false); });  // not a leaf
        Tensor li = Tensor::from_host(std::vector<int64_t>{1}, Shape({1}), kDev);
        ok = ok && throws([&] { li.set_requires_grad(); });    // int64
        return ok;
    });

    return g_failures == 0 ? 0 : 1;
}
