// SGD update over parameter/gradient tensor pairs (rule of
// legacy/include/dl/optim/Optimizer.hpp:24-34).
#include <dl/core/HipUtils.hpp>
#include <dl/kernels/sgd.hpp>
#include <dl/optim/SGD.hpp>

#include <hip/hip_runtime_api.h>

#include <stdexcept>

namespace dl::optim {

void SGD::step(const std::vector<Tensor*>& params, const std::vector<const Tensor*>& grads) const {
    if (params.size() != grads.size()) {
        throw std::runtime_error("SGD::step: parameter and gradient counts differ");
    }
    for (std::size_t i = 0; i < params.size(); ++i) {
        Tensor* p = params[i];
        const Tensor* g = grads[i];
        if (!p || !g || !p->defined() || !g->defined()) {
            throw std::runtime_error("SGD::step: undefined parameter or gradient");
        }
        if (p->shape().dims != g->shape().dims || p->dtype() != DType::Float32 ||
            g->dtype() != DType::Float32) {
            throw std::runtime_error("SGD::step: parameter and gradient must be float32 of one shape");
        }
        hip::check(hipSetDevice(p->device().index), "cudaSetDevice failed");
        kernels::sgd_update(static_cast<float*>(p->data()), static_cast<const float*>(g->data()),
                            lr_, p->numel());
    }
}

void SGD::step(const std::vector<Tensor*>& params) const {
    std::vector<Tensor*> ps;
    std::vector<Tensor> gs;
    for (Tensor* p : params) {
        if (!p) throw std::runtime_error("SGD::step: null parameter");
        Tensor g = p->grad();
        if (!g.defined()) continue;
        ps.push_back(p);
        gs.push_back(std::move(g));
    }
    std::vector<const Tensor*> gp;
    for (const Tensor& g : gs) gp.push_back(&g);
    step(ps, gp);
}

void SGD::zero_grad(const std::vector<Tensor*>& params) {
    for (Tensor* p : params) {
        if (p) p->zero_grad();
    }
}

}  // namespace dl::optim
