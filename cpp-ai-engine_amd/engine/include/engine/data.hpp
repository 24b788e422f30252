// data.hpp -- host-side dataset readers of the reference's
// include/engine/data.hpp: the IDX format MNIST ships in, the MNIST file
// layout, and a byte-level character vocabulary for language models. They
// build host data and hand the engine ordinary Tensors (uploaded on first
// use); nothing here touches the GPU.
#ifndef ENGINE_DATA_HPP
#define ENGINE_DATA_HPP

#include <cstddef>
#include <optional>
#include <string>
#include <vector>

#include "engine/tensor.hpp"

namespace engine {
namespace data {

// IDX files: a big-endian header (magic 0x00000803 for images, 0x00000801 for
// labels, then one int32 per axis) and unsigned bytes. Images come back as
// (N, 1, height, width) scaled to [0, 1]; max_samples > 0 keeps the first ones.
Tensor load_idx_images(const std::string& path, size_t max_samples = 0);
std::vector<size_t> load_idx_labels(const std::string& path, size_t max_samples = 0);

// The distinct bytes of a corpus in ascending (unsigned) order, each mapped to
// its position. encode drops bytes the corpus never had; decode drops indices
// past the alphabet.
class CharVocab {
public:
    explicit CharVocab(const std::string& corpus);

    size_t size() const noexcept { return symbols_.size(); }
    char symbol(size_t index) const { return symbols_.at(index); }
    std::optional<size_t> index_of(char symbol) const;
    std::vector<size_t> encode(const std::string& text) const;
    std::string decode(const std::vector<size_t>& indices) const;

private:
    std::string symbols_;
    std::vector<int> position_ = std::vector<int>(256, -1);  // byte -> index, -1 if absent
};

// The files' contents in the given order, each followed by a newline; a file
// that cannot be opened is reported on stderr and skipped.
std::string load_text(const std::vector<std::string>& paths);

struct Dataset {
    Tensor images;               // (N, 1, 28, 28)
    std::vector<size_t> labels;  // N
    size_t size() const { return labels.size(); }
};

struct MnistPaths {
    std::string train_images;
    std::string train_labels;
    std::string test_images;
    std::string test_labels;
    bool full = false;  // the whole set, or the reference repository's subset
};

// The full set's file names in `directory` if they are there, else the
// subset's ("subset-" prefixed); throws if neither is.
MnistPaths find_mnist(const std::string& directory = "data/mnist");
Dataset load_mnist_train(const MnistPaths& paths, size_t max_samples = 0);
Dataset load_mnist_test(const MnistPaths& paths, size_t max_samples = 0);

}  // namespace data
}  // namespace engine

#endif  // ENGINE_DATA_HPP
