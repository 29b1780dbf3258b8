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

Tensor Tensor::ones(std::vector<int64_t> shape, DType dtype) {
    return full(std::move(shape), 1.0f, dtype);
}

// One element uploaded, then broadcast by a strided copy with zero source
// strides.
Tensor Tensor::full(std::vector<int64_t> shape, float value, DType dtype) {
    Tensor t = empty(std::move(shape), dtype);
    if (t.numel_ == 0) return t;
    Tensor one = empty({1}, dtype);
    if (dtype == DType::Float16) {
        const __half h = __float2half(value);
        one.copy_from_cpu(&h, sizeof h);
    } else {
        one.copy_from_cpu(&value, sizeof value);
    }
    const std::vector<int64_t> zero(t.shape_.size(), 0);
    check_abi(msst_strided_copy(one.data_, zero.data(), t.data_, t.strides_.data(),
                                t.shape_.data(), t.ndim(), (int)dtype_size(dtype),
                                CudaContext::instance().stream()),
              "Tensor::full");
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

// tensor.cu:656-665: row-major strides, size-1 axes ignored.
bool Tensor::is_contiguous() const {
    if (numel_ <= 1) return true;
    int64_t expected = 1;
    for (int i = ndim() - 1; i >= 0; --i) {
        if (shape_[i] != 1 && strides_[i] != expected) return false;
        expected *= shape_[i];
    }
    return true;
}

void Tensor::copy_from_cpu(const void* src, size_t bytes) {
    if (!is_contiguous()) throw std::runtime_error("Tensor::copy_from_cpu: not contiguous");
    if (bytes > nbytes()) throw std::runtime_error("Tensor::copy_from_cpu: too many bytes");
    if (bytes == 0) return;
    hipStream_t s = CudaContext::instance().stream();
    HIP_CHECK(hipMemcpyAsync(data_, src, bytes, hipMemcpyHostToDevice, s));
    HIP_CHECK(hipStreamSynchronize(s));
}

void Tensor::copy_to_cpu(void* dst, size_t bytes) const {
    if (!is_contiguous()) {
        contiguous().copy_to_cpu(dst, bytes);
        return;
    }
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
    Tensor t = is_contiguous() ? *this : contiguous();
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
    if (shape_[d] != 1)
        throw std::runtime_error("Tensor::squeeze: dimension " + std::to_string(dim) + " of " +
                                 shape_str() + " is not 1");
    std::vector<int64_t> s = shape_;
    s.erase(s.begin() + d);
    return reshape(s);
}

// tensor.cu:837-855: the same storage with reordered shape and strides.
Tensor Tensor::permute(std::vector<int> dims) const {
    const int n = ndim();
    if ((int)dims.size() != n)
        throw std::runtime_error("Tensor::permute: " + std::to_string(dims.size()) +
                                 " dims for a " + std::to_string(n) + "-D tensor");
    std::vector<bool> seen(n, false);
    Tensor t = *this;
    for (int i = 0; i < n; ++i) {
        int d = dims[i] < 0 ? dims[i] + n : dims[i];
        if (d < 0 || d >= n || seen[d])
            throw std::runtime_error("Tensor::permute: dims are not a permutation");
        seen[d] = true;
        t.shape_[i] = shape_[d];
        t.strides_[i] = strides_[d];
    }
    return t;
}

Tensor Tensor::transpose(int dim0, int dim1) const {
    const int n = ndim();
    const int a = dim0 < 0 ? dim0 + n : dim0, b = dim1 < 0 ? dim1 + n : dim1;
    if (a < 0 || a >= n || b < 0 || b >= n)
        throw std::out_of_range("Tensor::transpose: dim out of range");
    std::vector<int> dims(n);
    for (int i = 0; i < n; ++i) dims[i] = i;
    std::swap(dims[a], dims[b]);
    return permute(dims);
}

// tensor.cu:868-903: one strided-copy launch into a new row-major tensor.
Tensor Tensor::contiguous() const {
    if (is_contiguous()) return *this;
    Tensor t = empty(shape_, dtype_);
    t.copy_from(*this);
    return t;
}

// tensor.cu:924-957: broadcast view, stride 0 along expanded axes (new
// leading axes allowed).
Tensor Tensor::expand(std::vector<int64_t> new_shape) const {
    const int n = (int)new_shape.size(), k = ndim();
    if (n < k) throw std::runtime_error("Tensor::expand: cannot drop dimensions");
    Tensor t = *this;
    t.shape_ = new_shape;
    t.strides_.assign(n, 0);
    t.numel_ = 1;
    for (int i = 0; i < n; ++i) {
        const int j = i - (n - k);  // aligned source axis
        const int64_t src = j >= 0 ? shape_[j] : 1;
        if (new_shape[i] == -1 && j >= 0) t.shape_[i] = src;
        if (t.shape_[i] < 0) throw std::runtime_error("Tensor::expand: negative extent");
        if (j >= 0 && src == t.shape_[i])
            t.strides_[i] = strides_[j];
        else if (src != 1)
            throw std::runtime_error("Tensor::expand: " + shape_str() + " cannot expand to axis " +
                                     std::to_string(i) + " of extent " +
                                     std::to_string(t.shape_[i]));
        t.numel_ *= t.shape_[i];
    }
    return t;
}

// tensor.cu:960-979: view of [start, end) along dim.
Tensor Tensor::slice(int dim, int64_t start, int64_t end) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("Tensor::slice: dim out of range");
    const int64_t ext = shape_[d];
    if (start < 0) start += ext;
    if (end < 0) end += ext;
    start = std::max<int64_t>(start, 0);
    end = std::min<int64_t>(end, ext);
    if (start >= end) return Tensor();
    Tensor t = *this;
    t.shape_[d] = end - start;
    t.numel_ = numel_ / ext * (end - start);
    t.data_ = static_cast<char*>(data_) + start * strides_[d] * (int64_t)dtype_size(dtype_);
    return t;
}

std::vector<Tensor> Tensor::split(int dim, const std::vector<int64_t>& sizes) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("Tensor::split: dim out of range");
    int64_t total = 0;
    for (int64_t s : sizes) total += s;
    if (total != shape_[d])
        throw std::runtime_error("Tensor::split: sizes sum to " + std::to_string(total) +
                                 ", dimension has " + std::to_string(shape_[d]));
    std::vector<Tensor> out;
    int64_t off = 0;
    for (int64_t s : sizes) {
        out.push_back(slice(d, off, off + s));
        off += s;
    }
    return out;
}

std::vector<Tensor> Tensor::unbind(int dim) const {
    const int n = ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("Tensor::unbind: dim out of range");
    std::vector<Tensor> out;
    for (int64_t i = 0; i < shape_[d]; ++i) out.push_back(slice(d, i, i + 1).squeeze(d));
    return out;
}

// tensor.cu:1062-1136: each input copied (strided, in place of the
// reference's contiguous() + slab kernel) into its slab of the output.
Tensor Tensor::cat(const std::vector<Tensor>& tensors, int dim) {
    if (tensors.empty()) throw std::runtime_error("Tensor::cat: empty tensor list");
    const Tensor& t0 = tensors[0];
    const int n = t0.ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("Tensor::cat: dim out of range");
    std::vector<int64_t> shape = t0.shape_;
    int64_t total = 0;
    for (const Tensor& t : tensors) {
        if (t.ndim() != n) throw std::runtime_error("Tensor::cat: ndim mismatch");
        if (t.dtype_ != t0.dtype_) throw std::runtime_error("Tensor::cat: dtype mismatch");
        for (int i = 0; i < n; ++i)
            if (i != d && t.shape_[i] != shape[i])
                throw std::runtime_error("Tensor::cat: shape " + t.shape_str() + " vs " +
                                         t0.shape_str());
        total += t.shape_[d];
    }
    shape[d] = total;
    Tensor out = empty(shape, t0.dtype_);
    int64_t off = 0;
    for (const Tensor& t : tensors) {
        if (t.numel_ > 0) out.slice(d, off, off + t.shape_[d]).copy_from(t);
        off += t.shape_[d];
    }
    return out;
}

// tensor.cu:1138-1150: unsqueeze every input at dim, then cat.
Tensor Tensor::stack(const std::vector<Tensor>& tensors, int dim) {
    if (tensors.empty()) throw std::runtime_error("Tensor::stack: empty tensor list");
    const int n = tensors[0].ndim() + 1;
    const int d = dim < 0 ? dim + n : dim;
    std::vector<Tensor> u;
    u.reserve(tensors.size());
    for (const Tensor& t : tensors) {
        // A view with a size-1 axis (no copy, unlike unsqueeze of a view).
        if (d < 0 || d > t.ndim()) throw std::out_of_range("Tensor::stack: dim out of range");
        Tensor v = t;
        v.shape_.insert(v.shape_.begin() + d, 1);
        v.strides_.insert(v.strides_.begin() + d, 0);
        u.push_back(v);
    }
    return cat(u, d);
}

Tensor Tensor::to_dtype(DType new_dtype) const {
    if (new_dtype == dtype_) return *this;
    if (!is_contiguous()) return contiguous().to_dtype(new_dtype);
    Tensor t = empty(shape_, new_dtype);
    if (numel_ > 0)
        check_abi(msst_cast(data_, abi_dtype(dtype_), t.data_, abi_dtype(new_dtype), numel_,
                            CudaContext::instance().stream()),
                  "Tensor::to_dtype");
    return t;
}

namespace {

// Broadcast shape of a and b (trailing-axis alignment, size-1 axes), or
// throws.
std::vector<int64_t> broadcast_shape(const std::vector<int64_t>& a, const std::vector<int64_t>& b,
                                     const char* what) {
    const size_t n = std::max(a.size(), b.size());
    std::vector<int64_t> out(n);
    for (size_t i = 0; i < n; ++i) {
        const int64_t x = i + a.size() >= n ? a[i + a.size() - n] : 1;
        const int64_t y = i + b.size() >= n ? b[i + b.size() - n] : 1;
        if (x != y && x != 1 && y != 1)
            throw std::runtime_error(std::string(what) + ": shapes do not broadcast");
        out[i] = x == 1 ? y : x;
    }
    return out;
}

// Element strides of t viewed at `shape` (t's axes aligned to the end;
// stride 0 along broadcast axes).
std::vector<int64_t> broadcast_strides(const Tensor& t, const std::vector<int64_t>& shape) {
    const size_t n = shape.size(), k = (size_t)t.ndim();
    std::vector<int64_t> s(n, 0);
    for (size_t i = n - k; i < n; ++i) {
        const size_t j = i - (n - k);
        s[i] = t.shape()[j] == 1 ? 0 : t.strides()[j];
    }
    return s;
}

}  // namespace

Tensor Tensor::binary(const Tensor& other, int op, const char* what) const {
    if (other.dtype_ != dtype_) throw std::runtime_error(std::string(what) + ": dtype mismatch");
    const std::vector<int64_t> shape = broadcast_shape(shape_, other.shape_, what);
    if ((int)shape.size() > 8) throw std::runtime_error(std::string(what) + ": more than 8 dims");
    Tensor t = empty(shape, dtype_);
    if (t.numel_ == 0) return t;
    if (op == MSST_BIN_ADD && shape_ == other.shape_ && is_contiguous() && other.is_contiguous()) {
        check_abi(msst_add(data_, other.data_, t.data_, abi_dtype(dtype_), numel_,
                           CudaContext::instance().stream()),
                  what);
        return t;
    }
    const std::vector<int64_t> sa = broadcast_strides(*this, shape);
    const std::vector<int64_t> sb = broadcast_strides(other, shape);
    check_abi(msst_binary(data_, sa.data(), other.data_, sb.data(), t.data_, shape.data(),
                          (int)shape.size(), op, abi_dtype(dtype_), CudaContext::instance().stream()),
              what);
    return t;
}

void Tensor::binary_inplace(const Tensor& other, int op, const char* what) {
    if (other.dtype_ != dtype_) throw std::runtime_error(std::string(what) + ": dtype mismatch");
    if (broadcast_shape(shape_, other.shape_, what) != shape_)
        throw std::runtime_error(std::string(what) + ": " + other.shape_str() +
                                 " does not broadcast to " + shape_str());
    if (numel_ == 0) return;
    if (!is_contiguous()) {
        // In place on a view: compute into a contiguous temporary, write back.
        Tensor t = binary(other, op, what);
        copy_from(t);
        return;
    }
    if (op == MSST_BIN_ADD && shape_ == other.shape_ && other.is_contiguous()) {
        check_abi(msst_add(data_, other.data_, data_, abi_dtype(dtype_), numel_,
                           CudaContext::instance().stream()),
                  what);
        return;
    }
    const std::vector<int64_t> sb = broadcast_strides(other, shape_);
    check_abi(msst_binary(data_, strides_.data(), other.data_, sb.data(), data_, shape_.data(),
                          ndim(), op, abi_dtype(dtype_), CudaContext::instance().stream()),
              what);
}

Tensor Tensor::operator+(const Tensor& other) const { return binary(other, MSST_BIN_ADD, "Tensor::operator+"); }
Tensor Tensor::operator-(const Tensor& other) const { return binary(other, MSST_BIN_SUB, "Tensor::operator-"); }
Tensor Tensor::operator*(const Tensor& other) const { return binary(other, MSST_BIN_MUL, "Tensor::operator*"); }
Tensor Tensor::operator/(const Tensor& other) const { return binary(other, MSST_BIN_DIV, "Tensor::operator/"); }

Tensor& Tensor::add_(const Tensor& other) {
    binary_inplace(other, MSST_BIN_ADD, "Tensor::add_");
    return *this;
}

Tensor& Tensor::mul_(const Tensor& other) {
    binary_inplace(other, MSST_BIN_MUL, "Tensor::mul_");
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
    if (numel_ == 0) return;
    if (is_contiguous() && src.is_contiguous()) {
        HIP_CHECK(hipMemcpyAsync(data_, src.data_, nbytes(), hipMemcpyDeviceToDevice,
                                 CudaContext::instance().stream()));
        return;
    }
    // Strided on either side: same shape required (the element order of a
    // view is its index order).
    if (src.shape_ != shape_)
        throw std::runtime_error("Tensor::copy_from: shape " + src.shape_str() + " vs " +
                                 shape_str());
    if (ndim() > 8) throw std::runtime_error("Tensor::copy_from: more than 8 dims");
    check_abi(msst_strided_copy(src.data_, src.strides_.data(), data_, strides_.data(),
                                shape_.data(), ndim(), (int)dtype_size(dtype_),
                                CudaContext::instance().stream()),
              "Tensor::copy_from");
}

std::string Tensor::shape_str() const {
    std::ostringstream o;
    o << "[";
    for (size_t i = 0; i < shape_.size(); ++i) o << (i ? ", " : "") << shape_[i];
    o << "]";
    return o.str();
}

}  // namespace cudasep
