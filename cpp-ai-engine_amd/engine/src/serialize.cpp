// serialize.cpp -- the checkpoint container (the reference's src/serialize.cpp
// format) over device-resident tensors, and Adam's state.
#include "engine/serialize.hpp"

#include <cstring>
#include <fstream>
#include <iterator>
#include <map>
#include <set>
#include <stdexcept>

#include "detail.hpp"

namespace engine {

using namespace detail;

namespace {

const char kMagic[8] = {'C', 'P', 'P', 'A', 'I', 'E', 'N', 'G'};

void need_little_endian() {
    const uint16_t probe = 1;
    unsigned char low = 0;
    std::memcpy(&low, &probe, 1);
    if (low != 1) throw std::runtime_error("checkpoint files are little-endian; this host is not");
}

struct Writer {
    std::ofstream out;
    std::string path;
    template <typename T>
    void raw(const T& v) {
        out.write(reinterpret_cast<const char*>(&v), sizeof(T));
    }
    void bytes(const void* p, size_t n) {
        out.write(static_cast<const char*>(p), static_cast<std::streamsize>(n));
    }
};

// The tensor's values on the host: one device-to-host copy straight from the
// device buffer when that holds the current values (no host mirror is made).
std::vector<float> values_of(const Tensor& t) {
    std::vector<float> v(t.size());
    if (t.size() == 0) return v;
    if (t.storage().resident_on_device()) {
        hip::check(ehip_memcpy_d2h(v.data(), t.storage().device(), v.size() * sizeof(float),
                                   nullptr),
                   "checkpoint read");
    } else {
        std::memcpy(v.data(), t.data(), v.size() * sizeof(float));
    }
    return v;
}

void write_file(const NamedTensors& tensors, const std::string& path) {
    need_little_endian();
    std::set<std::string> names;
    for (const auto& nt : tensors)
        if (!names.insert(nt.first).second)
            throw std::runtime_error("checkpoint: the name '" + nt.first +
                                     "' appears twice; a load could not tell them apart");
    Writer w;
    w.path = path;
    w.out.open(path, std::ios::binary | std::ios::trunc);
    if (!w.out) throw std::runtime_error("checkpoint: cannot open '" + path + "' for writing");
    w.bytes(kMagic, sizeof(kMagic));
    w.raw<uint32_t>(kSerializationVersion);
    w.raw<uint32_t>(static_cast<uint32_t>(tensors.size()));
    for (const auto& nt : tensors) {
        w.raw<uint32_t>(static_cast<uint32_t>(nt.first.size()));
        w.bytes(nt.first.data(), nt.first.size());
        const std::vector<size_t>& shape = nt.second.shape();
        w.raw<uint32_t>(static_cast<uint32_t>(shape.size()));
        for (size_t d : shape) w.raw<uint64_t>(static_cast<uint64_t>(d));
        const std::vector<float> v = values_of(nt.second);
        w.bytes(v.data(), v.size() * sizeof(float));
    }
    w.out.flush();
    if (!w.out) throw std::runtime_error("checkpoint: writing '" + path + "' failed");
}

struct Entry {
    std::string name;
    std::vector<size_t> shape;
    std::vector<float> values;
};

// Parses the whole file with every length checked against the bytes left, so
// a truncated or hostile file ends in an exception, never a wild read.
std::vector<Entry> read_file(const std::string& path) {
    need_little_endian();
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("checkpoint: cannot open '" + path + "'");
    const std::vector<char> buf((std::istreambuf_iterator<char>(in)),
                                std::istreambuf_iterator<char>());
    size_t at = 0;
    const auto left = [&] { return buf.size() - at; };
    const auto take = [&](void* dst, size_t n, const char* what) {
        if (n > left())
            throw std::runtime_error("checkpoint: '" + path + "' ends inside " + what);
        std::memcpy(dst, buf.data() + at, n);
        at += n;
    };
    char magic[sizeof(kMagic)];
    if (left() < sizeof(magic) || (take(magic, sizeof(magic), "the magic"),
                                   std::memcmp(magic, kMagic, sizeof(kMagic)) != 0))
        throw std::runtime_error("checkpoint: '" + path + "' is not a CPPAIENG weight file");
    uint32_t version = 0, count = 0;
    take(&version, 4, "the header");
    if (version != kSerializationVersion)
        throw std::runtime_error("checkpoint: '" + path + "' has format version " +
                                 std::to_string(version) + "; this build reads version " +
                                 std::to_string(kSerializationVersion));
    take(&count, 4, "the header");
    // Each entry needs at least 8 bytes (name length and rank).
    if (uint64_t(count) * 8 > left())
        throw std::runtime_error("checkpoint: '" + path + "' announces " + std::to_string(count) +
                                 " tensors, more than its size allows");
    std::vector<Entry> out;
    out.reserve(count);
    for (uint32_t t = 0; t < count; ++t) {
        Entry e;
        uint32_t name_len = 0, rank = 0;
        take(&name_len, 4, "a name length");
        if (name_len > left())
            throw std::runtime_error("checkpoint: '" + path + "' ends inside a tensor name");
        e.name.assign(buf.data() + at, name_len);
        at += name_len;
        take(&rank, 4, "a rank");
        if (uint64_t(rank) * 8 > left())
            throw std::runtime_error("checkpoint: '" + path + "' ends inside the shape of '" +
                                     e.name + "'");
        uint64_t total = 1;
        for (uint32_t d = 0; d < rank; ++d) {
            uint64_t dim = 0;
            take(&dim, 8, "a shape");
            if (dim != 0 && total > UINT64_MAX / dim)
                throw std::runtime_error("checkpoint: the shape of '" + e.name +
                                         "' overflows 64 bits");
            total *= dim;
            e.shape.push_back(static_cast<size_t>(dim));
        }
        if (total > left() / sizeof(float))
            throw std::runtime_error("checkpoint: '" + path + "' ends inside the values of '" +
                                     e.name + "'");
        e.values.resize(static_cast<size_t>(total));
        take(e.values.data(), e.values.size() * sizeof(float), "values");
        out.push_back(std::move(e));
    }
    return out;
}

std::string shape_text(const std::vector<size_t>& s) {
    std::string t = "(";
    for (size_t i = 0; i < s.size(); ++i) t += (i ? ", " : "") + std::to_string(s[i]);
    return t + ")";
}

// Host values into the tensor's device buffer (H2D); the host mirror goes stale.
void put_values(Tensor& t, const std::vector<float>& v) {
    if (v.empty()) return;
    hip::check(ehip_memcpy_h2d(t.storage().device_write(), v.data(), v.size() * sizeof(float),
                               nullptr),
               "checkpoint write");
}

}  // namespace

void save_parameters(const NamedTensors& params, const std::string& path) {
    write_file(params, path);
}

void save_parameters(nn::Module& model, const std::string& path) {
    write_file(model.named_parameters(), path);
}

size_t load_parameters(NamedTensors& params, const std::string& path, bool strict) {
    std::set<std::string> names;
    for (const auto& nt : params)
        if (!names.insert(nt.first).second)
            throw std::runtime_error("checkpoint: the name '" + nt.first + "' appears twice");
    const std::vector<Entry> stored = read_file(path);
    std::map<std::string, const Entry*> by_name;
    for (const Entry& e : stored) by_name[e.name] = &e;
    size_t loaded = 0;
    for (auto& nt : params) {
        auto it = by_name.find(nt.first);
        if (it == by_name.end()) {
            if (strict)
                throw std::runtime_error("checkpoint: '" + path + "' has no tensor '" + nt.first +
                                         "'");
            continue;
        }
        const Entry& e = *it->second;
        if (e.shape != nt.second.shape())
            throw std::runtime_error("checkpoint: '" + nt.first + "' is " +
                                     shape_text(nt.second.shape()) + " in the model and " +
                                     shape_text(e.shape) + " in '" + path + "'");
        put_values(nt.second, e.values);
        by_name.erase(it);
        ++loaded;
    }
    if (strict && !by_name.empty())
        throw std::runtime_error("checkpoint: '" + path + "' carries '" + by_name.begin()->first +
                                 "', which the model does not have");
    return loaded;
}

size_t load_parameters(nn::Module& model, const std::string& path, bool strict) {
    NamedTensors params = model.named_parameters();
    return load_parameters(params, path, strict);
}

std::vector<std::pair<std::string, std::vector<size_t>>> inspect_parameters(
    const std::string& path) {
    std::vector<std::pair<std::string, std::vector<size_t>>> out;
    for (const Entry& e : read_file(path)) out.emplace_back(e.name, e.shape);
    return out;
}

NamedTensors load_tensors(const std::string& path) {
    NamedTensors out;
    for (const Entry& e : read_file(path)) {
        Tensor t(e.shape, 0.0f, false);
        put_values(t, e.values);
        out.emplace_back(e.name, t);
    }
    return out;
}

void save_optimizer(const optim::Adam& opt, const std::string& path) {
    const size_t t = opt.steps();
    Tensor step({2}, 0.0f, false);
    put_values(step, {static_cast<float>(t % (size_t(1) << 24)),
                      static_cast<float>(t >> 24)});
    NamedTensors out{{"adam.t", step}};
    const std::vector<Tensor> moments = opt.state_tensors();
    for (size_t i = 0; i < moments.size(); ++i)
        out.emplace_back(std::string(i % 2 == 0 ? "adam.m." : "adam.v.") + std::to_string(i / 2),
                         moments[i]);
    write_file(out, path);
}

void load_optimizer(optim::Adam& opt, const std::string& path) {
    const std::vector<Entry> stored = read_file(path);
    std::map<std::string, const Entry*> by_name;
    for (const Entry& e : stored) by_name[e.name] = &e;
    auto step = by_name.find("adam.t");
    if (step == by_name.end() || step->second->values.size() != 2)
        throw std::runtime_error("checkpoint: '" + path + "' holds no Adam step count");
    const size_t t = static_cast<size_t>(step->second->values[0]) +
                     (static_cast<size_t>(step->second->values[1]) << 24);
    const size_t n = opt.state_tensors().size();
    std::vector<Tensor> moments;
    moments.reserve(n);
    for (size_t i = 0; i < n; ++i) {
        const std::string name =
            std::string(i % 2 == 0 ? "adam.m." : "adam.v.") + std::to_string(i / 2);
        auto it = by_name.find(name);
        if (it == by_name.end())
            throw std::runtime_error("checkpoint: '" + path + "' has no tensor '" + name + "'");
        Tensor m(it->second->shape, 0.0f, false);
        put_values(m, it->second->values);
        moments.push_back(m);
    }
    opt.set_state(t, moments);
}

}  // namespace engine
