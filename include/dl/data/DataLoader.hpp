#pragma once
// MNIST IDX loader: the reference's legacy DataLoader
// (legacy/include/dl/data/DataLoader.hpp, legacy/src/data/DataLoader.cpp)
// with the same constructor, size queries and per-record label access, and
// with the images delivered as GPU tensors instead of an Eigen matrix.
//
// The files are read once on the host.  The raw bytes (one byte per pixel and
// per label) are uploaded to a device on first use and stay there; every
// float32 image tensor is produced on the GPU from those bytes as
// pixel / 255.0f, bit for bit the value the reference computes on the host.
// A training batch is one gather launch from the resident bytes.

#include <cstdint>
#include <string>
#include <vector>

#include <dl/core/Device.hpp>
#include <dl/tensor/Tensor.hpp>

namespace dl::data {

class DataLoader {
public:
    // Reads an IDX3 image file (magic 0x803: count, rows, cols, then
    // count*rows*cols pixel bytes) and an IDX1 label file (magic 0x801:
    // count, then count label bytes).  num > 0 keeps the first num records of
    // each file (DataLoader.cpp:43,85); num == 0 keeps all.  Throws
    // std::runtime_error for a file that cannot be opened
    // ("Could not open image file: <path>", DataLoader.cpp:30; the label
    // file gets the same check), a wrong magic number or a truncated file
    // (where the reference asserts or reads past the end), and for num < 0.
    DataLoader(std::string image_file, std::string label_file, int num);
    DataLoader(std::string image_file, std::string label_file);
    ~DataLoader();

    int getSize() const { return size_; }   // image records kept
    int getRows() const { return rows_; }
    int getCols() const { return cols_; }

    // Label of record id, as the reference reads it: the byte through a
    // signed char (DataLoader.cpp:88-90).  Throws std::out_of_range for an
    // id outside the label records.
    int getLabels(int id) const;
    int label_count() const { return static_cast<int>(labels_.size()); }

    // float32 [getSize(), rows*cols] = pixel / 255.0f, computed on `device`
    // (the reference's getImagesMatrix).
    Tensor getImagesMatrix(const Device& device = Device(DeviceType::CUDA, 0));
    // float32 [1, rows*cols]: record idx (getImageRow).  Throws
    // std::out_of_range for idx outside [0, getSize()).
    Tensor getImageRow(int idx, const Device& device = Device(DeviceType::CUDA, 0));
    // int64 [label_count()] on `device`.
    Tensor labels(const Device& device = Device(DeviceType::CUDA, 0));

    // One batch: for b in [0, batch), record r = index[start + b] goes to
    // x[b, :] (float32 [batch, rows*cols], pixel / 255.0f) and y[b] (int64
    // [batch]).  index is an int64 device tensor of record numbers (e.g. from
    // permutation()); x, y and index live on one device, where the bytes are
    // uploaded on first use.  Records must be < min(getSize(), label_count());
    // an index the loader did not make is checked on the device: an entry out
    // of range gives a zero row and label -1.  Runs on the current stream.
    void gather(const Tensor& index, int64_t start, int64_t batch, Tensor& x, Tensor& y);

    // int64 [getSize()] on `device`: a permutation of 0..getSize()-1, a
    // Fisher-Yates shuffle driven by std::mt19937_64(seed) on the host (an
    // epoch order; the reference has no shuffling).
    Tensor permutation(uint64_t seed, const Device& device = Device(DeviceType::CUDA, 0)) const;

    // The raw bytes as read (row-major pixels; labels).
    const std::vector<uint8_t>& pixel_bytes() const { return pixels_; }
    const std::vector<uint8_t>& label_bytes() const { return labels_; }

private:
    void upload(const Device& device);

    std::vector<uint8_t> pixels_;
    std::vector<uint8_t> labels_;
    int size_ = 0;
    int rows_ = 0;
    int cols_ = 0;
    // Device copies of pixels_ and labels_ (byte storage), made on first use.
    Tensor device_pixels_;
    Tensor device_labels_;
};

}  // namespace dl::data
