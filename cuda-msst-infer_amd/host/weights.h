// weights.h — the reference's converted-checkpoint container (".csm",
// src/weights.h:98-118, loader weights.cu:412-508):
//
//   "CSM\0"  u32 version (1)  u32 config_len  config JSON (UTF-8)
//   u32 num_tensors, then per tensor:
//     u32 name_len, name, u32 ndim, i64 shape[ndim], u32 dtype (0 f32,
//     1 f16, 2 i64), raw little-endian data (numel * dtype size bytes)
//
// Tensors go to device memory as they are read.  convert_linear_weights_to_fp16
// is the reference's --fp16 load step (weights.cu:510-524): every 2-D fp32
// tensor becomes fp16.
#pragma once

#include <map>
#include <string>
#include <vector>

#include "json.h"
#include "tensor.h"

namespace cudasep {

class ModelWeights {
public:
    static ModelWeights load(const std::string& path);

    const JsonValue& config() const { return config_; }
    bool has(const std::string& name) const { return tensors_.count(name) != 0; }
    const Tensor& get(const std::string& name) const;  // throws if missing
    std::vector<std::string> names() const;
    size_t size() const { return tensors_.size(); }

    void convert_linear_weights_to_fp16();

private:
    JsonValue config_;
    std::map<std::string, Tensor> tensors_;
};

}  // namespace cudasep
