#pragma once
// One training epoch of train::Mlp2 from an IDX set resident on the GPU
// (data::DataLoader): full batches in a given record order, each fed to one
// fused training step.
//
// By default the epoch's batches are gathered together, in one launch, into
// an fp32 buffer of steps * batch rows (188 MB for MNIST's 60000 records at
// batch 256), and each step reads its rows at an offset.  One gather of the
// whole order streams at HBM speed where a gather per step costs a launch
// per step.  Running the per-step gathers on a second stream beside the steps
// was measured slower on MI355X: each step then waits on an event from the
// other stream, which costs more than the gather it hides.
// whole_epoch = false gathers before each step into one batch buffer.  The
// arithmetic is the same either way, so the trained weights are identical.

#include <cstdint>

#include <dl/data/DataLoader.hpp>
#include <dl/tensor/Tensor.hpp>
#include <dl/train/Mlp2.hpp>

namespace dl::train {

struct EpochResult {
    int64_t steps = 0;       // full batches trained (a last partial batch is dropped)
    float last_loss = 0.0f;  // mean loss of the last step
};

// order: int64 device tensor of record numbers (e.g. loader.permutation(seed));
// the net's input width must match the loader's records.  Runs on the
// current stream and synchronises once at the end to read the last loss.
EpochResult train_epoch(Mlp2& net, data::DataLoader& loader, const Tensor& order, float lr,
                        bool whole_epoch = true);

}  // namespace dl::train
