// weights.cpp — .csm reader (format in weights.h).
#include "weights.h"

#include <cstring>
#include <fstream>
#include <stdexcept>

namespace cudasep {

ModelWeights ModelWeights::load(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("ModelWeights: cannot open " + path);
    auto bytes = [&](void* dst, size_t n) {
        f.read(reinterpret_cast<char*>(dst), (std::streamsize)n);
        if (!f) throw std::runtime_error("ModelWeights: truncated file " + path);
    };
    auto u32 = [&]() {
        uint32_t v;
        bytes(&v, 4);
        return v;
    };
    char magic[4];
    bytes(magic, 4);
    if (std::memcmp(magic, "CSM\0", 4) != 0)
        throw std::runtime_error("ModelWeights: not a .csm file (magic) " + path);
    const uint32_t version = u32();
    if (version != 1)
        throw std::runtime_error("ModelWeights: unsupported version " + std::to_string(version));
    std::string cfg(u32(), '\0');
    if (!cfg.empty()) bytes(&cfg[0], cfg.size());

    ModelWeights w;
    w.config_ = JsonValue::parse(cfg);
    const uint32_t count = u32();
    std::vector<char> buf;
    for (uint32_t t = 0; t < count; ++t) {
        std::string name(u32(), '\0');
        if (!name.empty()) bytes(&name[0], name.size());
        const uint32_t ndim = u32();
        if (ndim > 8) throw std::runtime_error("ModelWeights: tensor " + name + " has ndim > 8");
        std::vector<int64_t> shape(ndim);
        int64_t numel = 1;
        for (uint32_t d = 0; d < ndim; ++d) {
            bytes(&shape[d], 8);
            if (shape[d] < 0) throw std::runtime_error("ModelWeights: negative dim in " + name);
            numel *= shape[d];
        }
        const uint32_t code = u32();
        if (code > 2)
            throw std::runtime_error("ModelWeights: unknown dtype " + std::to_string(code) +
                                     " for " + name);
        const DType dt = code == 0 ? DType::Float32 : code == 1 ? DType::Float16 : DType::Int64;
        Tensor tensor = Tensor::empty(shape, dt);
        const size_t nb = (size_t)numel * dtype_size(dt);
        if (nb > 0) {
            buf.resize(nb);
            bytes(buf.data(), nb);
            tensor.copy_from_cpu(buf.data(), nb);
        }
        w.tensors_[name] = tensor;
    }
    return w;
}

const Tensor& ModelWeights::get(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("ModelWeights: tensor not found: " + name);
    return it->second;
}

std::vector<std::string> ModelWeights::names() const {
    std::vector<std::string> n;
    for (const auto& kv : tensors_) n.push_back(kv.first);
    return n;
}

void ModelWeights::convert_linear_weights_to_fp16() {
    for (auto& kv : tensors_)
        if (kv.second.ndim() == 2 && kv.second.dtype() == DType::Float32)
            kv.second = kv.second.to_f16();
}

}  // namespace cudasep
