#pragma once
// Umbrella header of the dl:: API (reference include/dl/dl.hpp).

#include <dl/autograd/Node.hpp>
#include <dl/core/DType.hpp>
#include <dl/core/Device.hpp>
#include <dl/core/Shape.hpp>
#include <dl/core/Stream.hpp>
#include <dl/data/DataLoader.hpp>
#include <dl/nn/Linear.hpp>
#include <dl/nn/Module.hpp>
#include <dl/nn/ReLU.hpp>
#include <dl/nn/Sequential.hpp>
#include <dl/ops/Ops.hpp>
#include <dl/optim/SGD.hpp>
#include <dl/tensor/Tensor.hpp>
#include <dl/train/Epoch.hpp>
#include <dl/train/Mlp2.hpp>
