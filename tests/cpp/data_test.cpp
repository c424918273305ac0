// dl::data::DataLoader checks on the GPU, in the reference's test style: each
// check prints "<name> : passed|not passed" and the program exits non-zero if
// any fails.  IDX files are written here byte by byte from the published
// format; the host expression static_cast<float>(p) / 255.0f is the
// reference's own conversion (legacy/src/data/DataLoader.cpp:65-66) and is the
// checker for the GPU-converted tensors.
#include <dl/dl.hpp>

#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <limits>
#include <numeric>
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

void put_word(std::vector<uint8_t>& out, uint32_t v) {
    out.push_back(uint8_t(v >> 24));
    out.push_back(uint8_t(v >> 16));
    out.push_back(uint8_t(v >> 8));
    out.push_back(uint8_t(v));
}

void write_file(const std::string& path, const std::vector<uint8_t>& bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(reinterpret_cast<const char*>(bytes.data()), static_cast<std::streamsize>(bytes.size()));
}

void write_idx3(const std::string& path, int n, int rows, int cols, const std::vector<uint8_t>& px,
                uint32_t magic = 0x803, std::size_t truncate = 0) {
    std::vector<uint8_t> b;
    put_word(b, magic);
    put_word(b, uint32_t(n));
    put_word(b, uint32_t(rows));
    put_word(b, uint32_t(cols));
    b.insert(b.end(), px.begin(), px.end());
    b.resize(b.size() - truncate);
    write_file(path, b);
}

void write_idx1(const std::string& path, const std::vector<uint8_t>& labels, uint32_t magic = 0x801,
                std::size_t truncate = 0) {
    std::vector<uint8_t> b;
    put_word(b, magic);
    put_word(b, uint32_t(labels.size()));
    b.insert(b.end(), labels.begin(), labels.end());
    b.resize(b.size() - truncate);
    write_file(path, b);
}

std::vector<uint8_t> random_bytes(std::size_t n, uint32_t seed, int hi = 255) {
    std::mt19937 gen(seed);
    std::uniform_int_distribution<int> d(0, hi);
    std::vector<uint8_t> v(n);
    for (auto& x : v) x = uint8_t(d(gen));
    return v;
}

bool same_bits(const std::vector<float>& a, const std::vector<float>& b) {
    return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

// The reference's conversion of one pixel (DataLoader.cpp:65-66).
float ref_pixel(uint8_t p) { return static_cast<float>(p) / 255.0f; }

std::string exe_dir() {
    char buf[4096];
    const ssize_t n = readlink("/proc/self/exe", buf, sizeof(buf) - 1);
    if (n <= 0) return ".";
    buf[n] = 0;
    std::string s(buf);
    return s.substr(0, s.find_last_of('/'));
}

const dl::Device kDev(dl::DeviceType::CUDA, 0);

}  // namespace

int main() {
    char tmpl[] = "/tmp/fdl_data_test_XXXXXX";
    const char* dir_c = mkdtemp(tmpl);
    if (!dir_c) {
        std::cout << "mkdtemp failed" << std::endl;
        return 1;
    }
    const std::string dir(dir_c);
    const std::string img = dir + "/images", lab = dir + "/labels";

    // 300 images of 28x28 with random bytes; labels 0..9 plus bytes >= 128.
    const int n = 300, rows = 28, cols = 28, px = rows * cols;
    const std::vector<uint8_t> pixels = random_bytes(std::size_t(n) * px, 11);
    std::vector<uint8_t> labels = random_bytes(n, 12, 9);
    labels[3] = 200;
    labels[4] = 128;
    write_idx3(img, n, rows, cols, pixels);
    write_idx1(lab, labels);

    run("idx_loader_reads_sizes_labels_and_num_limit", [&] {
        dl::data::DataLoader all(img, lab);
        dl::data::DataLoader some(img, lab, 17);
        bool ok = all.getSize() == n && all.getRows() == rows && all.getCols() == cols &&
                  all.label_count() == n && some.getSize() == 17 && some.label_count() == 17;
        ok = ok && all.getLabels(3) == -56 && all.getLabels(4) == -128;  // signed char reads
        for (int i = 0; i < n; ++i) ok = ok && all.getLabels(i) == int(int8_t(labels[i]));
        ok = ok && dl::data::DataLoader(img, lab, 100000).getSize() == n;
        return ok && all.pixel_bytes() == pixels;
    });

    run("images_matrix_is_the_reference_conversion_bit_for_bit", [&] {
        dl::data::DataLoader d(img, lab);
        const Tensor x = d.getImagesMatrix(kDev);
        std::vector<float> want(pixels.size());
        for (std::size_t i = 0; i < pixels.size(); ++i) want[i] = ref_pixel(pixels[i]);
        return x.shape()[0] == n && x.shape()[1] == px && same_bits(x.to_host<float>(), want);
    });

    run("image_row_and_labels_tensor", [&] {
        dl::data::DataLoader d(img, lab);
        bool ok = true;
        for (int i : {0, 1, 150, n - 1}) {
            const std::vector<float> row = d.getImageRow(i, kDev).to_host<float>();
            std::vector<float> want(px);
            for (int j = 0; j < px; ++j) want[j] = ref_pixel(pixels[std::size_t(i) * px + j]);
            ok = ok && same_bits(row, want);
        }
        const std::vector<int64_t> y = d.labels(kDev).to_host<int64_t>();
        for (int i = 0; i < n; ++i) ok = ok && y[i] == d.getLabels(i);
        return ok;
    });

    run("permutation_batches_cover_an_epoch_on_a_stream", [&] {
        dl::data::DataLoader d(img, lab);
        const Tensor perm = d.permutation(7, kDev);
        std::vector<int64_t> order = perm.to_host<int64_t>();
        std::vector<int64_t> sorted = order;
        std::sort(sorted.begin(), sorted.end());
        std::vector<int64_t> iota(n);
        std::iota(iota.begin(), iota.end(), int64_t(0));
        bool ok = sorted == iota && order != iota;
        ok = ok && d.permutation(7, kDev).to_host<int64_t>() == order &&
             d.permutation(8, kDev).to_host<int64_t>() != order;
        dl::Stream stream(kDev);
        dl::StreamGuard guard(stream);
        const int B = 64;
        for (int start = 0; start < n; start += B) {
            const int b = std::min(B, n - start);  // the last batch is ragged
            Tensor x(Shape({b, px}), DType::Float32, kDev), y(Shape({b}), DType::Int64, kDev);
            d.gather(perm, start, b, x, y);
            const std::vector<float> xh = x.to_host<float>();
            const std::vector<int64_t> yh = y.to_host<int64_t>();
            for (int r = 0; r < b; ++r) {
                const int64_t rec = order[start + r];
                ok = ok && yh[r] == int64_t(int8_t(labels[rec]));
                for (int j = 0; j < px; ++j) {
                    const float want = ref_pixel(pixels[rec * px + j]);
                    ok = ok && std::memcmp(&xh[std::size_t(r) * px + j], &want, 4) == 0;
                }
            }
        }
        return ok;
    });

    run("bad_files_and_arguments_throw", [&] {
        const std::string missing = dir + "/nope";
        bool ok = message_of([&] { dl::data::DataLoader(missing, lab); }) ==
                  "Could not open image file: " + missing;
        ok = ok && message_of([&] { dl::data::DataLoader(img, missing); }) ==
                       "Could not open label file: " + missing;
        const std::string bad = dir + "/bad";
        write_idx3(bad, n, rows, cols, pixels, 0x801);
        ok = ok && message_of([&] { dl::data::DataLoader(bad, lab); }).rfind("Bad magic", 0) == 0;
        write_idx3(bad, n, rows, cols, pixels, 0x803, 1);
        ok = ok && message_of([&] { dl::data::DataLoader(bad, lab); }).rfind("Truncated", 0) == 0;
        write_idx1(bad, labels, 0x801, 1);
        ok = ok && message_of([&] { dl::data::DataLoader(img, bad); }).rfind("Truncated", 0) == 0;
        ok = ok && !message_of([&] { dl::data::DataLoader(img, lab, -1); }).empty();
        dl::data::DataLoader d(img, lab);
        ok = ok && !message_of([&] { d.getLabels(n); }).empty() &&
             !message_of([&] { d.getImageRow(-1, kDev); }).empty();
        const Tensor perm = d.permutation(1, kDev);
        Tensor x(Shape({8, px}), DType::Float32, kDev), y(Shape({8}), DType::Int64, kDev);
        ok = ok && message_of([&] { d.gather(perm, n - 4, 8, x, y); }).find("outside index") !=
                       std::string::npos;
        Tensor xw(Shape({8, px + 1}), DType::Float32, kDev);
        ok = ok && !message_of([&] { d.gather(perm, 0, 8, xw, y); }).empty();
        return ok;
    });

    run("out_of_range_index_gives_zero_row_and_label_minus_one", [&] {
        dl::data::DataLoader d(img, lab);
        const Tensor index = Tensor::from_host(std::vector<int64_t>{5, -1, n, 2}, Shape({4}), kDev);
        Tensor x(Shape({4, px}), DType::Float32, kDev), y(Shape({4}), DType::Int64, kDev);
        d.gather(index, 0, 4, x, y);
        const std::vector<float> xh = x.to_host<float>();
        const std::vector<int64_t> yh = y.to_host<int64_t>();
        bool ok = yh[1] == -1 && yh[2] == -1 && yh[0] == int8_t(labels[5]) && yh[3] == int8_t(labels[2]);
        for (int j = 0; j < px; ++j) {
            ok = ok && xh[std::size_t(px) + j] == 0.0f && xh[std::size_t(2) * px + j] == 0.0f &&
                 xh[j] == ref_pixel(pixels[std::size_t(5) * px + j]);
        }
        return ok;
    });

    run("reference_mnist_label_file", [&] {
        // The reference's train labels (a fixture of this repository) with
        // small synthetic images of the same count.
        const std::string labels_path = exe_dir() + "/../../golden/mnist/train-labels-idx1-ubyte";
        const std::string small = dir + "/small_images";
        write_idx3(small, 60000, 2, 2, random_bytes(60000 * 4, 13));
        dl::data::DataLoader d(small, labels_path);
        const int counts[10] = {5923, 6742, 5958, 6131, 5842, 5421, 5918, 6265, 5851, 5949};
        const int first[10] = {5, 0, 4, 1, 9, 2, 1, 3, 1, 4};
        const std::vector<int64_t> y = d.labels(kDev).to_host<int64_t>();
        int hist[10] = {0};
        bool ok = d.getSize() == 60000 && d.label_count() == 60000 && int(y.size()) == 60000;
        for (int64_t v : y) {
            ok = ok && v >= 0 && v < 10;
            if (v >= 0 && v < 10) ++hist[v];
        }
        for (int c = 0; c < 10; ++c) ok = ok && hist[c] == counts[c] && d.getLabels(c) == first[c];
        return ok;
    });

    run("mlp_trains_from_resident_batches", [&] {
        // 4 classes of 8x8 images: class c is bright in rows 2c..2c+1.
        const int N = 2048, R = 8, C = 8, P = R * C, classes = 4, B = 128;
        std::vector<uint8_t> px_bytes(std::size_t(N) * P), lab_bytes(N);
        std::mt19937 gen(21);
        std::uniform_int_distribution<int> noise(0, 60), cls(0, classes - 1);
        for (int i = 0; i < N; ++i) {
            const int c = cls(gen);
            lab_bytes[i] = uint8_t(c);
            for (int j = 0; j < P; ++j) {
                const bool hot = j / C / 2 == c;
                px_bytes[std::size_t(i) * P + j] = uint8_t(noise(gen) + (hot ? 180 : 0));
            }
        }
        const std::string ti = dir + "/train_images", tl = dir + "/train_labels";
        write_idx3(ti, N, R, C, px_bytes);
        write_idx1(tl, lab_bytes);
        dl::data::DataLoader d(ti, tl);
        dl::train::Mlp2 net(P, 32, classes, B, kDev, 3);
        Tensor x(Shape({B, P}), DType::Float32, kDev), y(Shape({B}), DType::Int64, kDev);
        float first_loss = 0, last_loss = 0;
        for (int epoch = 0; epoch < 4; ++epoch) {
            const Tensor perm = d.permutation(100 + epoch, kDev);
            for (int start = 0; start + B <= N; start += B) {
                d.gather(perm, start, B, x, y);
                const float loss = net.step(x, y, 0.2f);
                if (epoch == 0 && start == 0) first_loss = loss;
                last_loss = loss;
            }
        }
        std::cout << "  loss " << first_loss << " -> " << last_loss << std::endl;
        return std::isfinite(last_loss) && last_loss < 0.25f * first_loss;
    });

    run("whole_epoch_gather_trains_to_the_per_batch_bits", [&] {
        // 60000 synthetic 28x28 records with the reference's labels, batch 256:
        // one gather for the epoch or one per step, the same arithmetic.
        const std::string labels_path = exe_dir() + "/../../golden/mnist/train-labels-idx1-ubyte";
        const std::string big = dir + "/epoch_images";
        write_idx3(big, 60000, 28, 28, random_bytes(std::size_t(60000) * 784, 31));
        dl::data::DataLoader d(big, labels_path);
        const Tensor order = d.permutation(5, kDev);
        dl::train::Mlp2 a(784, 256, 10, 256, kDev, 17), b(784, 256, 10, 256, kDev, 17);
        const auto t0 = std::chrono::steady_clock::now();
        const dl::train::EpochResult ra = dl::train::train_epoch(a, d, order, 0.05f, true);
        const auto t1 = std::chrono::steady_clock::now();
        const dl::train::EpochResult rb = dl::train::train_epoch(b, d, order, 0.05f, false);
        const auto t2 = std::chrono::steady_clock::now();
        const auto bits = [](const Tensor& p, const Tensor& q) {
            const std::vector<float> x = p.to_host<float>(), y = q.to_host<float>();
            return std::memcmp(x.data(), y.data(), x.size() * sizeof(float)) == 0;
        };
        const double ms_a = std::chrono::duration<double, std::milli>(t1 - t0).count();
        const double ms_b = std::chrono::duration<double, std::milli>(t2 - t1).count();
        std::cout << "  epoch of " << ra.steps << " steps: whole-epoch gather " << ms_a
                  << " ms, per-batch gathers " << ms_b << " ms (first epoch, includes the upload)"
                  << std::endl;
        std::remove(big.c_str());
        return ra.steps == 234 && rb.steps == 234 && ra.last_loss == rb.last_loss &&
               std::isfinite(ra.last_loss) && bits(a.w1(), b.w1()) && bits(a.b1(), b.b1()) &&
               bits(a.w2(), b.w2()) && bits(a.b2(), b.b2());
    });

    // best-effort cleanup of the temporary files
    for (const char* f : {"/images", "/labels", "/bad", "/small_images", "/train_images",
                          "/train_labels"}) {
        std::remove((dir + f).c_str());
    }
    rmdir(dir.c_str());
    return g_failures == 0 ? 0 : 1;
}
