// MNIST IDX loader over fdl_idx_gather.  File parsing follows
// legacy/src/data/DataLoader.cpp:22-93 of the reference (big-endian header
// words, the num limit, one byte per pixel and per label); the float
// conversion runs on the GPU.
#include <dl/core/HipUtils.hpp>
#include <dl/core/Stream.hpp>
#include <dl/data/DataLoader.hpp>

#include <fastdl_data.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <fstream>
#include <limits>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <utility>

namespace dl::data {

namespace {

constexpr int kImageMagic = 0x803;
constexpr int kLabelMagic = 0x801;
constexpr float kPixelDivisor = 255.0f;

// One big-endian 32-bit header word (DataLoader.cpp:22-25).
int32_t read_word(std::ifstream& in, const std::string& path) {
    unsigned char p[4];
    if (!in.read(reinterpret_cast<char*>(p), 4)) {
        throw std::runtime_error("Truncated IDX header in " + path);
    }
    const uint32_t v = (uint32_t(p[0]) << 24) | (uint32_t(p[1]) << 16) | (uint32_t(p[2]) << 8) |
                       uint32_t(p[3]);
    return static_cast<int32_t>(v);
}

void read_bytes(std::ifstream& in, std::vector<uint8_t>& out, const std::string& path) {
    if (!out.empty() &&
        !in.read(reinterpret_cast<char*>(out.data()), static_cast<std::streamsize>(out.size()))) {
        throw std::runtime_error("Truncated IDX data in " + path);
    }
}

// The record count after the num limit (DataLoader.cpp:43,85).
int32_t limit(int32_t count, int num, const std::string& path) {
    if (count < 0) throw std::runtime_error("Negative record count in " + path);
    return (num != 0 && num < count) ? num : count;
}

const uint8_t* u8(const Tensor& t) { return static_cast<const uint8_t*>(t.data()); }

}  // namespace

DataLoader::DataLoader(std::string image_file, std::string label_file, int num) {
    if (num < 0) throw std::runtime_error("DataLoader: num must be >= 0");
    {
        std::ifstream in(image_file, std::ios::in | std::ios::binary);
        if (!in) throw std::runtime_error("Could not open image file: " + image_file);
        if (read_word(in, image_file) != kImageMagic) {
            throw std::runtime_error("Bad magic number in image file: " + image_file);
        }
        size_ = limit(read_word(in, image_file), num, image_file);
        rows_ = read_word(in, image_file);
        cols_ = read_word(in, image_file);
        if (rows_ < 0 || cols_ < 0) throw std::runtime_error("Negative image size in " + image_file);
        const uint64_t n = uint64_t(size_) * uint64_t(rows_) * uint64_t(cols_);
        if (n > uint64_t(std::numeric_limits<int64_t>::max() / 4)) {
            throw std::runtime_error("Image file too large: " + image_file);
        }
        pixels_.resize(static_cast<std::size_t>(n));
        read_bytes(in, pixels_, image_file);
    }
    {
        std::ifstream in(label_file, std::ios::in | std::ios::binary);
        if (!in) throw std::runtime_error("Could not open label file: " + label_file);
        if (read_word(in, label_file) != kLabelMagic) {
            throw std::runtime_error("Bad magic number in label file: " + label_file);
        }
        labels_.resize(static_cast<std::size_t>(limit(read_word(in, label_file), num, label_file)));
        read_bytes(in, labels_, label_file);
    }
}

DataLoader::DataLoader(std::string image_file, std::string label_file)
    : DataLoader(std::move(image_file), std::move(label_file), 0) {}

DataLoader::~DataLoader() = default;

int DataLoader::getLabels(int id) const {
    if (id < 0 || id >= label_count()) throw std::out_of_range("DataLoader::getLabels: id out of range");
    return static_cast<int>(static_cast<int8_t>(labels_[static_cast<std::size_t>(id)]));
}

void DataLoader::upload(const Device& device) {
    if (!device.is_cuda()) throw std::runtime_error("DataLoader: device must be a GPU");
    const bool have = device_pixels_.defined() || device_labels_.defined();
    const bool same = have && (device_pixels_.defined() ? device_pixels_ : device_labels_)
                                      .device().index == device.index;
    if (same) return;
    device_pixels_ = Tensor();
    device_labels_ = Tensor();
    // Byte storage: DType::Bool is the API's one-byte element type.
    if (!pixels_.empty()) {
        device_pixels_ = Tensor(Shape({static_cast<int64_t>(pixels_.size())}), DType::Bool, device);
        device_pixels_.copy_from_host(pixels_.data(), pixels_.size());
    }
    if (!labels_.empty()) {
        device_labels_ = Tensor(Shape({static_cast<int64_t>(labels_.size())}), DType::Bool, device);
        device_labels_.copy_from_host(labels_.data(), labels_.size());
    }
}

Tensor DataLoader::getImagesMatrix(const Device& device) {
    upload(device);
    const int64_t pixels = int64_t(rows_) * cols_;
    Tensor out(Shape({size_, pixels}), DType::Float32, device);
    if (out.numel() == 0) return out;
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    hip::check_fdl(fdl_idx_gather(u8(device_pixels_), nullptr, size_, pixels, nullptr, size_,
                                  kPixelDivisor, static_cast<float*>(out.data()), nullptr,
                                  current_stream()),
                   "DataLoader::getImagesMatrix failed");
    return out;
}

Tensor DataLoader::getImageRow(int idx, const Device& device) {
    if (idx < 0 || idx >= size_) throw std::out_of_range("DataLoader::getImageRow: idx out of range");
    upload(device);
    const int64_t pixels = int64_t(rows_) * cols_;
    Tensor out(Shape({1, pixels}), DType::Float32, device);
    if (pixels == 0) return out;
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    hip::check_fdl(fdl_idx_gather(u8(device_pixels_) + int64_t(idx) * pixels, nullptr, 1, pixels,
                                  nullptr, 1, kPixelDivisor, static_cast<float*>(out.data()),
                                  nullptr, current_stream()),
                   "DataLoader::getImageRow failed");
    return out;
}

Tensor DataLoader::labels(const Device& device) {
    upload(device);
    const int64_t n = label_count();
    Tensor out(Shape({n}), DType::Int64, device);
    if (n == 0) return out;
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    hip::check_fdl(fdl_idx_gather(nullptr, u8(device_labels_), n, 0, nullptr, n, kPixelDivisor,
                                  nullptr, static_cast<int64_t*>(out.data()), current_stream()),
                   "DataLoader::labels failed");
    return out;
}

void DataLoader::gather(const Tensor& index, int64_t start, int64_t batch, Tensor& x, Tensor& y) {
    const int64_t pixels = int64_t(rows_) * cols_;
    if (index.dtype() != DType::Int64 || index.shape().rank() != 1) {
        throw std::runtime_error("DataLoader::gather: index must be an int64 vector");
    }
    if (start < 0 || batch < 0 || start > index.numel() - batch) {
        throw std::runtime_error("DataLoader::gather: [start, start + batch) outside index");
    }
    if (x.dtype() != DType::Float32 || x.shape().rank() != 2 || x.shape()[0] != batch ||
        x.shape()[1] != pixels) {
        throw std::runtime_error("DataLoader::gather: x must be float32 [batch, rows*cols]");
    }
    if (y.dtype() != DType::Int64 || y.shape().rank() != 1 || y.shape()[0] != batch) {
        throw std::runtime_error("DataLoader::gather: y must be int64 [batch]");
    }
    const Device device = index.device();
    if (!device.is_cuda() || x.device().index != device.index || y.device().index != device.index ||
        !x.device().is_cuda() || !y.device().is_cuda()) {
        throw std::runtime_error("DataLoader::gather: index, x and y must be on one GPU");
    }
    if (batch == 0) return;
    upload(device);
    // Records beyond the shorter of the two files count as out of range.
    const int64_t count = std::min<int64_t>(size_, label_count());
    hip::check(hipSetDevice(device.index), "cudaSetDevice failed");
    hip::check_fdl(fdl_idx_gather(u8(device_pixels_), u8(device_labels_), count, pixels,
                                  static_cast<const int64_t*>(index.data()) + start, batch,
                                  kPixelDivisor, pixels ? static_cast<float*>(x.data()) : nullptr,
                                  static_cast<int64_t*>(y.data()), current_stream()),
                   "DataLoader::gather failed");
}

Tensor DataLoader::permutation(uint64_t seed, const Device& device) const {
    std::vector<int64_t> order(static_cast<std::size_t>(size_));
    std::iota(order.begin(), order.end(), int64_t(0));
    std::mt19937_64 gen(seed);
    for (std::size_t i = order.size(); i > 1; --i) {
        std::uniform_int_distribution<std::size_t> pick(0, i - 1);
        std::swap(order[i - 1], order[pick(gen)]);
    }
    return Tensor::from_host(order, Shape({size_}), device);
}

}  // namespace dl::data
