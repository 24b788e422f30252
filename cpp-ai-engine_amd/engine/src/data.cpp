// data.cpp -- IDX and MNIST readers, the character vocabulary and the corpus
// loader (the reference's src/data.cpp: file layouts and behaviour as there).
#include "engine/data.hpp"

#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iterator>
#include <stdexcept>

namespace engine {
namespace data {

namespace {

struct Idx {
    std::vector<uint32_t> dims;
    std::vector<unsigned char> bytes;  // the first `count` items
    size_t count = 0;                  // items read (along the first axis)
};

uint32_t big_endian(const unsigned char* p) {
    return (uint32_t(p[0]) << 24) | (uint32_t(p[1]) << 16) | (uint32_t(p[2]) << 8) | uint32_t(p[3]);
}

// Reads an IDX file of the given magic; keeps at most max_items items (0 =
// all) of the first axis.
Idx read_idx(const std::string& path, uint32_t magic, size_t max_items) {
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("Cannot open IDX file '" + path + "'.");
    unsigned char word[4];
    if (!in.read(reinterpret_cast<char*>(word), 4))
        throw std::runtime_error("IDX file '" + path + "' ends inside its header.");
    const uint32_t got = big_endian(word);
    if (got != magic)
        throw std::runtime_error("IDX file '" + path + "': magic " + std::to_string(got) +
                                 ", expected " + std::to_string(magic) + ".");
    Idx idx;
    const size_t ndims = magic & 0xffu;
    // The header's dimensions are untrusted: the payload size they imply is
    // checked for overflow and against the bytes the file still holds before
    // anything is allocated, so a corrupt header reads as a truncated file.
    const auto truncated = [&] {
        return std::runtime_error("IDX file '" + path + "' holds fewer than " +
                                  std::to_string(idx.count) + " items.");
    };
    size_t item = 1;
    bool overflow = false;
    for (size_t d = 0; d < ndims; ++d) {
        if (!in.read(reinterpret_cast<char*>(word), 4))
            throw std::runtime_error("IDX file '" + path + "' ends inside its header.");
        idx.dims.push_back(big_endian(word));
        if (d > 0) overflow |= __builtin_mul_overflow(item, size_t(idx.dims.back()), &item);
    }
    const size_t items = ndims ? idx.dims[0] : 0;
    idx.count = max_items > 0 && max_items < items ? max_items : items;
    size_t payload = 0;
    overflow |= __builtin_mul_overflow(idx.count, item, &payload);
    const std::streampos start = in.tellg();
    in.seekg(0, std::ios::end);
    const std::streampos end = in.tellg();
    in.seekg(start);
    if (overflow || start < 0 || end < start || payload > size_t(end - start)) throw truncated();
    idx.bytes.resize(payload);
    if (!in.read(reinterpret_cast<char*>(idx.bytes.data()), std::streamsize(idx.bytes.size())))
        throw truncated();
    return idx;
}

bool readable(const std::string& path) { return std::ifstream(path, std::ios::binary).good(); }

}  // namespace

// The IDX header check on its own, for the C ABI's tests: items kept and
// payload bytes of a file, or the reader's exception.
size_t idx_payload_bytes(const std::string& path, uint32_t magic, size_t max_items,
                         size_t* count) {
    const Idx idx = read_idx(path, magic, max_items);
    if (count) *count = idx.count;
    return idx.bytes.size();
}

Tensor load_idx_images(const std::string& path, size_t max_samples) {
    const Idx idx = read_idx(path, 0x00000803u, max_samples);
    if (idx.dims.size() != 3)
        throw std::runtime_error("IDX images in '" + path + "' are not 2-D.");
    std::vector<float> values(idx.bytes.size());
    for (size_t i = 0; i < values.size(); ++i) values[i] = float(idx.bytes[i]) / 255.0f;
    return Tensor({idx.count, 1, size_t(idx.dims[1]), size_t(idx.dims[2])}, values, false);
}

std::vector<size_t> load_idx_labels(const std::string& path, size_t max_samples) {
    const Idx idx = read_idx(path, 0x00000801u, max_samples);
    return std::vector<size_t>(idx.bytes.begin(), idx.bytes.end());
}

CharVocab::CharVocab(const std::string& corpus) {
    bool present[256] = {};
    for (const unsigned char c : corpus) present[c] = true;
    for (int b = 0; b < 256; ++b) {
        if (!present[b]) continue;
        position_[b] = int(symbols_.size());
        symbols_.push_back(char(b));
    }
}

std::optional<size_t> CharVocab::index_of(char symbol) const {
    const int at = position_[static_cast<unsigned char>(symbol)];
    if (at < 0) return std::nullopt;
    return size_t(at);
}

std::vector<size_t> CharVocab::encode(const std::string& text) const {
    std::vector<size_t> ids;
    ids.reserve(text.size());
    for (const char c : text)
        if (const auto at = index_of(c)) ids.push_back(*at);
    return ids;
}

std::string CharVocab::decode(const std::vector<size_t>& indices) const {
    std::string text;
    text.reserve(indices.size());
    for (const size_t i : indices)
        if (i < symbols_.size()) text.push_back(symbols_[i]);
    return text;
}

std::string load_text(const std::vector<std::string>& paths) {
    std::string corpus;
    for (const std::string& path : paths) {
        std::ifstream in(path, std::ios::binary);
        if (!in) {
            std::fprintf(stderr, "engine: skipping unreadable file %s\n", path.c_str());
            continue;
        }
        corpus.append(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
        corpus.push_back('\n');
    }
    return corpus;
}

MnistPaths find_mnist(const std::string& directory) {
    MnistPaths p;
    const auto fill = [&](const std::string& prefix, const std::string& test) {
        p.train_images = directory + "/" + prefix + "train-images-idx3-ubyte";
        p.train_labels = directory + "/" + prefix + "train-labels-idx1-ubyte";
        p.test_images = directory + "/" + prefix + test + "-images-idx3-ubyte";
        p.test_labels = directory + "/" + prefix + test + "-labels-idx1-ubyte";
    };
    fill("", "t10k");
    if (readable(p.train_images)) {
        p.full = true;
        return p;
    }
    fill("subset-", "test");
    if (readable(p.train_images)) return p;
    throw std::runtime_error("No MNIST files (full set or subset) in '" + directory + "'.");
}

Dataset load_mnist_train(const MnistPaths& paths, size_t max_samples) {
    return Dataset{load_idx_images(paths.train_images, max_samples),
                   load_idx_labels(paths.train_labels, max_samples)};
}

Dataset load_mnist_test(const MnistPaths& paths, size_t max_samples) {
    return Dataset{load_idx_images(paths.test_images, max_samples),
                   load_idx_labels(paths.test_labels, max_samples)};
}

}  // namespace data
}  // namespace engine
