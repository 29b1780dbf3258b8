// tensor.cpp — see tensor.h.
#include "tensor.h"

#include <algorithm>
#include <sstream>

#include "memory_pool.h"
#include "msst_hip.h"
#include "ops.h"

namespace cudasep {

namespace {

int abi_dtype(DType dt) {
    if (dt == DType::Float32) return MSST_F32;
    if (dt == DType::Float16) return MSST_F16;
    throw std::runtime_error("Tensor: int64 tensors have no device kernels on this path");
}

void check_abi(int rc, const char* what) {
    if (rc != MSST_OK) throw std::runtime_error(std::string(what) + ": " + msst_last_error());
}

}  // namespace

Tensor::Tensor() : data_(nullptr), numel_(0), dtype_(DType::Float32) {}

void Tensor::compute_strides() {
    strides_.assign(shape_.size(), 1);
    int64_t s = 1;
    for (int i = (int)shape_.size() - 1; i >= 0; --i) {
        strides_[i] = s;
        s *= shape_[i];
    }
    numel_ = s;
}

Tensor Tensor::empty(std::vector<int64_t> shape, DType dtype) {
    for (int64_t d : shape)
        if (d < 0) throw std::runtime_error("Tensor::empty: negative dimension");
    Tensor t;
    t.shape_ = std::move(shape);
    t.dtype_ = dtype;
    t.compute_strides();
    if (t.numel_ > 0) {
        void* p = DeviceMemoryPool::instance().allocate(t.nbytes());
        t.storage_ = std::shared_ptr<void>(p, [](void* q) { DeviceMemoryPool::instance().deallocate(q); });
        t.data_ = p;
    }
    return t;
}

Tensor Tensor::zeros(std::vector<int64_t> shape, DType dtype) {
    Tensor t = empty(std::move(shape), dtype);
    if (t.numel_ > 0)
        HIP_CHECK(hipMemsetAsync(t.data_, 0, t.nbytes(), CudaContext::instance().stream()));
    return t;
}

Tensor Tensor::from_cpu_f32(const float* data, std::vector<int64_t> shape) {
    Tensor t = empty(std::move(shape), DType::Float32);
    t.copy_from_cpu(data, t.nbytes());
    return t;
}

Tensor Tensor::from_cpu_f16(const void* data, std::vector<int64_t> shape) {
    Tensor t = empty(std::move(shape), DType::Float16);
    t.copy_from_cpu(data, t.nbytes());
    return t;
}

int64_t Tensor::size(int dim) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n)
        throw std::out_of_range("Tensor::size: dim " + std::to_string(dim) + " out of range for " +
                                shape_str());
    return shape_[d];
}

float* Tensor::data_f32() {
    if (dtype_ != DType::Float32) throw std::runtime_error("Tensor::data_f32 on a non-f32 tensor");
    return static_cast<float*>(data_);
}
const float* Tensor::data_f32() const {
    if (dtype_ != DType::Float32) throw std::runtime_error("Tensor::data_f32 on a non-f32 tensor");
    return static_cast<const float*>(data_);
}
__half* Tensor::data_f16() {
    if (dtype_ != DType::Float16) throw std::runtime_error("Tensor::data_f16 on a non-f16 tensor");
    return static_cast<__half*>(data_);
}
const __half* Tensor::data_f16() const {
    if (dtype_ != DType::Float16) throw std::runtime_error("Tensor::data_f16 on a non-f16 tensor");
    return static_cast<const __half*>(data_);
}

void Tensor::copy_from_cpu(const void* src, size_t bytes) {
    if (bytes > nbytes()) throw std::runtime_error("Tensor::copy_from_cpu: too many bytes");
    if (bytes == 0) return;
    hipStream_t s = CudaContext::instance().stream();
    HIP_CHECK(hipMemcpyAsync(data_, src, bytes, hipMemcpyHostToDevice, s));
    HIP_CHECK(hipStreamSynchronize(s));
}

void Tensor::copy_to_cpu(void* dst, size_t bytes) const {
    if (bytes > nbytes()) throw std::runtime_error("Tensor::copy_to_cpu: too many bytes");
    if (bytes == 0) return;
    hipStream_t s = CudaContext::instance().stream();
    HIP_CHECK(hipMemcpyAsync(dst, data_, bytes, hipMemcpyDeviceToHost, s));
    HIP_CHECK(hipStreamSynchronize(s));
}

std::vector<float> Tensor::to_cpu_f32() const {
    Tensor f = to_f32();
    std::vector<float> out((size_t)f.numel_);
    f.copy_to_cpu(out.data(), f.nbytes());
    return out;
}

Tensor Tensor::reshape(std::vector<int64_t> new_shape) const {
    int64_t known = 1;
    int infer = -1;
    for (size_t i = 0; i < new_shape.size(); ++i) {
        if (new_shape[i] == -1) {
            if (infer >= 0) throw std::runtime_error("Tensor::reshape: more than one -1");
            infer = (int)i;
        } else {
            known *= new_shape[i];
        }
    }
    if (infer >= 0) {
        if (known == 0 || numel_ % known != 0)
            throw std::runtime_error("Tensor::reshape: cannot infer -1 for " + shape_str());
        new_shape[infer] = numel_ / known;
        known *= new_shape[infer];
    }
    if (known != numel_)
        throw std::runtime_error("Tensor::reshape: " + shape_str() + " has " +
                                 std::to_string(numel_) + " elements");
    Tensor t = *this;
    t.shape_ = std::move(new_shape);
    t.compute_strides();
    return t;
}

Tensor Tensor::unsqueeze(int dim) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n + 1 : dim;
    if (d < 0 || d > n) throw std::out_of_range("Tensor::unsqueeze: dim out of range");
    std::vector<int64_t> s = shape_;
    s.insert(s.begin() + d, 1);
    return reshape(s);
}

Tensor Tensor::squeeze(int dim) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("Tensor::squeeze: dim out of range");
    if (shape_[d] != 1) return *this;
    std::vector<int64_t> s = shape_;
    s.erase(s.begin() + d);
    return reshape(s);
}

Tensor Tensor::to_dtype(DType new_dtype) const {
    if (new_dtype == dtype_) return *this;
    Tensor t = empty(shape_, new_dtype);
    if (numel_ > 0)
        check_abi(msst_cast(data_, abi_dtype(dtype_), t.data_, abi_dtype(new_dtype), numel_,
                            CudaContext::instance().stream()),
                  "Tensor::to_dtype");
    return t;
}

Tensor Tensor::operator+(const Tensor& other) const {
    if (other.dtype_ != dtype_) throw std::runtime_error("Tensor::operator+: dtype mismatch");
    if (other.shape_ != shape_)
        throw std::runtime_error("Tensor::operator+: shape " + shape_str() + " vs " +
                                 other.shape_str());
    Tensor t = empty(shape_, dtype_);
    if (numel_ > 0)
        check_abi(msst_add(data_, other.data_, t.data_, abi_dtype(dtype_), numel_,
                           CudaContext::instance().stream()),
                  "Tensor::operator+");
    return t;
}

Tensor& Tensor::add_(const Tensor& other) {
    if (other.dtype_ != dtype_) throw std::runtime_error("Tensor::add_: dtype mismatch");
    if (other.shape_ != shape_)
        throw std::runtime_error("Tensor::add_: shape " + shape_str() + " vs " +
                                 other.shape_str());
    if (numel_ > 0)
        check_abi(msst_add(data_, other.data_, data_, abi_dtype(dtype_), numel_,
                           CudaContext::instance().stream()),
                  "Tensor::add_");
    return *this;
}

Tensor Tensor::clone() const {
    Tensor t = empty(shape_, dtype_);
    t.copy_from(*this);
    return t;
}

void Tensor::copy_from(const Tensor& src) {
    if (src.numel_ != numel_ || src.dtype_ != dtype_)
        throw std::runtime_error("Tensor::copy_from: size or dtype mismatch");
    if (numel_ > 0)
        HIP_CHECK(hipMemcpyAsync(data_, src.data_, nbytes(), hipMemcpyDeviceToDevice,
                                 CudaContext::instance().stream()));
}

std::string Tensor::shape_str() const {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < shape_.size(); ++i) o << (i ? ", " : "") << shape_[i];
    o << "]";
    return o.str();
}

}  // namespace cudasep
