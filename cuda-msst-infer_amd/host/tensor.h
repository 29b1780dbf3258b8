// tensor.h — the reference `cudasep::Tensor` (src/tensor.h:36-143) as the
// Roformer path and its callers use it, on HIP device memory.
//
// Same names, shapes, dtype enum, view semantics and error behaviour as the
// reference: device errors and shape errors throw std::runtime_error, an
// out-of-range dimension throws std::out_of_range.  Storage is reference
// counted and comes from a caching device pool (memory_pool.h), so
// temporaries are recycled instead of hitting hipMalloc/hipFree.
//
// Views share storage (tensor.cu:837-979): permute / transpose / expand /
// slice / split / unbind only change shape, strides and the data offset.
// contiguous() of a strided view is one msst_strided_copy launch;
// reshape / squeeze / unsqueeze of a non-contiguous tensor copy first, as
// the reference's reshape does.  Binary operators broadcast (trailing-axis
// alignment, size-1 axes) and read strided operands in place
// (msst_binary).  Every cudasep::ops function accepts views: it works on
// contiguous() of its inputs.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

namespace cudasep {

enum class DType { Float32 = 0, Float16 = 1, Int64 = 2 };

inline size_t dtype_size(DType dt) {
    switch (dt) {
        case DType::Float32: return 4;
        case DType::Float16: return 2;
        case DType::Int64: return 8;
    }
    return 0;
}

// Device-call error check (the reference's CUDA_CHECK, src/tensor.h:28-34).
#define HIP_CHECK(call)                                                                   \
    do {                                                                                  \
        hipError_t err_ = (call);                                                         \
        if (err_ != hipSuccess)                                                           \
            throw std::runtime_error(std::string("HIP error: ") + hipGetErrorString(err_) + \
                                     " at " + __FILE__ + ":" + std::to_string(__LINE__));  \
    } while (0)

class Tensor {
public:
    Tensor();  // empty (numel 0, no storage)

    // Factories (device memory, current device).
    static Tensor empty(std::vector<int64_t> shape, DType dtype = DType::Float32);
    static Tensor zeros(std::vector<int64_t> shape, DType dtype = DType::Float32);
    static Tensor ones(std::vector<int64_t> shape, DType dtype = DType::Float32);
    static Tensor full(std::vector<int64_t> shape, float value, DType dtype = DType::Float32);
    static Tensor from_cpu_f32(const float* data, std::vector<int64_t> shape);
    static Tensor from_cpu_f16(const void* data, std::vector<int64_t> shape);

    // Properties
    int ndim() const { return (int)shape_.size(); }
    int64_t size(int dim) const;  // negative dims count from the end
    const std::vector<int64_t>& shape() const { return shape_; }
    const std::vector<int64_t>& strides() const { return strides_; }
    int64_t numel() const { return numel_; }
    DType dtype() const { return dtype_; }
    bool is_contiguous() const;  // row-major up to size-1 axes
    bool is_empty() const { return numel_ == 0; }
    size_t nbytes() const { return (size_t)numel_ * dtype_size(dtype_); }

    // Raw data access (dtype-checked: throws on a mismatch).
    void* data_ptr() { return data_; }
    const void* data_ptr() const { return data_; }
    float* data_f32();
    const float* data_f32() const;
    __half* data_f16();
    const __half* data_f16() const;

    // Host transfer (synchronous on the context stream).
    std::vector<float> to_cpu_f32() const;
    void copy_from_cpu(const void* src, size_t bytes);
    void copy_to_cpu(void* dst, size_t bytes) const;

    // Shape operations (views where the layout allows, as in the reference).
    Tensor reshape(std::vector<int64_t> new_shape) const;  // one -1 allowed
    Tensor permute(std::vector<int> dims) const;            // view
    Tensor transpose(int dim0, int dim1) const;             // view
    Tensor contiguous() const;  // *this when contiguous, else a strided copy
    Tensor unsqueeze(int dim) const;
    Tensor squeeze(int dim) const;  // throws unless size(dim) == 1
    Tensor expand(std::vector<int64_t> new_shape) const;    // broadcast view

    // Slicing: [start, end) along dim (negative indices count from the end,
    // clamped to the extent; an empty range gives an empty Tensor).
    Tensor slice(int dim, int64_t start, int64_t end) const;  // view

    // Concat / split.
    static Tensor cat(const std::vector<Tensor>& tensors, int dim);
    static Tensor stack(const std::vector<Tensor>& tensors, int dim);
    std::vector<Tensor> split(int dim, const std::vector<int64_t>& sizes) const;  // views
    std::vector<Tensor> unbind(int dim) const;

    // Type conversion (returns *this when the dtype already matches).
    Tensor to_dtype(DType new_dtype) const;
    Tensor to_f32() const { return to_dtype(DType::Float32); }
    Tensor to_f16() const { return to_dtype(DType::Float16); }

    // Elementwise with broadcasting (a dtype mismatch throws, as
    // src/tensor.cu:1374 does; fp16 is computed in fp32).  The in-place
    // forms broadcast `other` into this tensor's shape.
    Tensor operator+(const Tensor& other) const;
    Tensor operator-(const Tensor& other) const;
    Tensor operator*(const Tensor& other) const;
    Tensor operator/(const Tensor& other) const;
    Tensor& add_(const Tensor& other);
    Tensor& mul_(const Tensor& other);

    Tensor clone() const;             // contiguous copy
    void copy_from(const Tensor& src);  // same shape and dtype; either may be a view

    std::string shape_str() const;

private:
    std::shared_ptr<void> storage_;
    void* data_;
    std::vector<int64_t> shape_;
    std::vector<int64_t> strides_;
    int64_t numel_;
    DType dtype_;

    void compute_strides();
    Tensor binary(const Tensor& other, int op, const char* what) const;
    void binary_inplace(const Tensor& other, int op, const char* what);
};

}  // namespace cudasep
