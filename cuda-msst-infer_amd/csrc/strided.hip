// strided.hip — the device side of cudasep::Tensor's strided views
// (permute / transpose / slice / expand / split, host/tensor.cpp):
//   msst_strided_copy  dst[i] = src[i] over an index space, both sides
//                      addressed by element strides: contiguous() of a view
//                      and the slab copies of cat / stack (tensor.cu:868-903,
//                      :1062-1150)
//   msst_binary        out = a op b (+ - * /) with broadcast strides, out
//                      contiguous: Tensor operator+ - * / and add_ / mul_
//                      with broadcasting (tensor.cu:1365-1447)
// Both are HBM-bound.  The host merges the dimensions that are contiguous
// in every operand and drops size-1 ones, so the common views (a permute
// that keeps the innermost axis, a slice of rows) reduce to 2-3 axes; the
// innermost axis is then copied 16 bytes per lane when it is contiguous
// and 16-byte aligned everywhere.  Linear indices are split into
// coordinates with multiply-high division by the invariant extents
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994), not hardware-less 64-bit division.
#include <algorithm>

#include "msst_common.hpp"
#include "strided_index.hpp"

namespace msst {
namespace {

// One operand's strides (in elements) over the merged axes.
struct StrideSet {
    int64_t s[kMaxDims];
};

// Element of `bytes` bytes (1, 2, 4, 8 or 16 for the vector path).
template <int BYTES>
struct Elem;
template <>
struct Elem<1> { typedef uint8_t T; };
template <>
struct Elem<2> { typedef uint16_t T; };
template <>
struct Elem<4> { typedef uint32_t T; };
template <>
struct Elem<8> { typedef uint64_t T; };
template <>
struct Elem<16> { typedef u4v T; };

// Copy of `total` units (elements, or 16-byte vectors when the innermost
// axis was folded into vectors by the host) in grid-stride order over the
// destination index space.
template <int BYTES>
__global__ __launch_bounds__(256) void strided_copy_kernel(const char* __restrict__ src,
                                                           char* __restrict__ dst, IndexSpace sp,
                                                           StrideSet ss, StrideSet ds,
                                                           uint64_t total) {
    typedef typename Elem<BYTES>::T T;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        int64_t so = 0, d_o = 0;
        uint64_t rem = i;
#pragma unroll
        for (int d = kMaxDims - 1; d >= 0; --d) {
            if (d < sp.ndim) {
                uint64_t q;
                const uint64_t c = sp.div[d].divmod(rem, &q);
                rem = q;
                so += (int64_t)c * ss.s[d];
                d_o += (int64_t)c * ds.s[d];
            }
        }
        *reinterpret_cast<T*>(dst + d_o * BYTES) = *reinterpret_cast<const T*>(src + so * BYTES);
    }
}

template <typename T>
__device__ __forceinline__ float ld_f(const T* p);
template <>
__device__ __forceinline__ float ld_f<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float ld_f<half_t>(const half_t* p) { return (float)*p; }

template <int OP>
__device__ __forceinline__ float bin_op(float a, float b) {
    if constexpr (OP == MSST_BIN_ADD) return a + b;
    else if constexpr (OP == MSST_BIN_SUB) return a - b;
    else if constexpr (OP == MSST_BIN_MUL) return a * b;
    else return a / b;
}

// out[i] = a[i] op b[i] over the merged index space, out contiguous.  VEC
// outputs per lane along the innermost axis (VEC = 4 when the innermost
// extent is a multiple of 4 and out is 4-element aligned; a and b then
// step by their own innermost stride, which is 1 or 0).
template <typename T, int OP, int VEC>
__global__ __launch_bounds__(256) void binary_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                     T* out, IndexSpace sp, StrideSet as,
                                                     StrideSet bs, uint64_t total) {
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    const int inner = sp.ndim - 1;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += step) {
        int64_t ao = 0, bo = 0;
        uint64_t rem = i;
#pragma unroll
        for (int d = kMaxDims - 1; d >= 0; --d) {
            if (d < sp.ndim) {
                uint64_t q;
                uint64_t c = sp.div[d].divmod(rem, &q);
                rem = q;
                if (d == inner) c *= VEC;
                ao += (int64_t)c * as.s[d];
                bo += (int64_t)c * bs.s[d];
            }
        }
        const int64_t sa = as.s[inner], sb = bs.s[inner];
#pragma unroll
        for (int v = 0; v < VEC; ++v)
            out[i * VEC + v] = (T)bin_op<OP>(ld_f<T>(a + ao + v * sa), ld_f<T>(b + bo + v * sb));
    }
}

int grid_for(uint64_t total) {
    const uint64_t blocks = (total + 255) / 256;
    return (int)std::min<uint64_t>(std::max<uint64_t>(blocks, 1), 8192);
}

template <typename T, int OP>
void launch_binary(const void* a, const void* b, void* out, const IndexSpace& sp,
                   const StrideSet& as, const StrideSet& bs, uint64_t total, int vec,
                   hipStream_t s) {
    const T* pa = reinterpret_cast<const T*>(a);
    const T* pb = reinterpret_cast<const T*>(b);
    T* po = reinterpret_cast<T*>(out);
    if (vec == 4)
        hipLaunchKernelGGL((binary_kernel<T, OP, 4>), dim3(grid_for(total)), dim3(256), 0, s, pa,
                           pb, po, sp, as, bs, total);
    else
        hipLaunchKernelGGL((binary_kernel<T, OP, 1>), dim3(grid_for(total)), dim3(256), 0, s, pa,
                           pb, po, sp, as, bs, total);
}

template <typename T>
void launch_binary_op(int op, const void* a, const void* b, void* out, const IndexSpace& sp,
                      const StrideSet& as, const StrideSet& bs, uint64_t total, int vec,
                      hipStream_t s) {
    switch (op) {
        case MSST_BIN_ADD: launch_binary<T, MSST_BIN_ADD>(a, b, out, sp, as, bs, total, vec, s); break;
        case MSST_BIN_SUB: launch_binary<T, MSST_BIN_SUB>(a, b, out, sp, as, bs, total, vec, s); break;
        case MSST_BIN_MUL: launch_binary<T, MSST_BIN_MUL>(a, b, out, sp, as, bs, total, vec, s); break;
        default: launch_binary<T, MSST_BIN_DIV>(a, b, out, sp, as, bs, total, vec, s); break;
    }
}

bool args_ok(const int64_t* shape, int ndim, std::initializer_list<const int64_t*> strides) {
    if (!shape || ndim < 0 || ndim > kMaxDims) return false;
    for (int d = 0; d < ndim; ++d)
        if (shape[d] < 0) return false;
    for (const int64_t* s : strides) {
        if (!s && ndim > 0) return false;
        for (int d = 0; d < ndim; ++d)
            if (s[d] < 0) return false;
    }
    return true;
}

}  // namespace
}  // namespace msst

extern "C" int msst_strided_copy(const void* src, const int64_t* src_strides, void* dst,
                                 const int64_t* dst_strides, const int64_t* shape, int ndim,
                                 int elem_bytes, void* stream) {
    using namespace msst;
    MSST_REQUIRE(args_ok(shape, ndim, {src_strides, dst_strides}), MSST_ERR_INVALID_ARG,
                 "ndim must be 0..8 with non-negative extents and strides");
    MSST_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
                 MSST_ERR_INVALID_ARG, "elem_bytes must be 1, 2, 4 or 8");
    MergedAxes m = merge_axes(shape, ndim, {src_strides, dst_strides});
    if (m.empty) return MSST_OK;
    MSST_REQUIRE(src && dst, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(aligned(src, elem_bytes) && aligned(dst, elem_bytes), MSST_ERR_ALIGNMENT,
                 "pointers must be aligned to the element size");
    hipStream_t s = as_stream(stream);
    // 16-byte vectors along a contiguous innermost axis.
    const int in = m.ndim - 1;
    const int per = 16 / elem_bytes;
    bool vec = m.stride[0][in] == 1 && m.stride[1][in] == 1 && m.shape[in] % per == 0 &&
               aligned(src, 16) && aligned(dst, 16);
    for (int d = 0; vec && d < in; ++d)
        vec = (m.stride[0][d] * elem_bytes) % 16 == 0 && (m.stride[1][d] * elem_bytes) % 16 == 0;
    int bytes = elem_bytes;
    if (vec) {
        m.shape[in] /= per;
        for (int d = 0; d < in; ++d) {
            m.stride[0][d] /= per;
            m.stride[1][d] /= per;
        }
        bytes = 16;
    }
    IndexSpace sp;
    uint64_t total = 0;
    MSST_REQUIRE(make_index_space(m, sp, total), MSST_ERR_UNSUPPORTED,
                 "index space exceeds 2^62 elements");
    StrideSet ss{}, ds{};
    for (int d = 0; d < m.ndim; ++d) {
        ss.s[d] = m.stride[0][d];
        ds.s[d] = m.stride[1][d];
    }
    const char* cs = reinterpret_cast<const char*>(src);
    char* cd = reinterpret_cast<char*>(dst);
    const dim3 g(grid_for(total)), b(256);
    switch (bytes) {
        case 1: hipLaunchKernelGGL(strided_copy_kernel<1>, g, b, 0, s, cs, cd, sp, ss, ds, total); break;
        case 2: hipLaunchKernelGGL(strided_copy_kernel<2>, g, b, 0, s, cs, cd, sp, ss, ds, total); break;
        case 4: hipLaunchKernelGGL(strided_copy_kernel<4>, g, b, 0, s, cs, cd, sp, ss, ds, total); break;
        case 8: hipLaunchKernelGGL(strided_copy_kernel<8>, g, b, 0, s, cs, cd, sp, ss, ds, total); break;
        default: hipLaunchKernelGGL(strided_copy_kernel<16>, g, b, 0, s, cs, cd, sp, ss, ds, total);
    }
    return check_launch("strided_copy_kernel");
}

extern "C" int msst_binary(const void* a, const int64_t* a_strides, const void* b,
                           const int64_t* b_strides, void* out, const int64_t* shape, int ndim,
                           int op, int dtype, void* stream) {
    using namespace msst;
    MSST_REQUIRE(args_ok(shape, ndim, {a_strides, b_strides}), MSST_ERR_INVALID_ARG,
                 "ndim must be 0..8 with non-negative extents and strides");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "dtype must be MSST_F32 or MSST_F16");
    MSST_REQUIRE(op >= MSST_BIN_ADD && op <= MSST_BIN_DIV, MSST_ERR_INVALID_ARG, "unknown op");
    // out is contiguous over `shape`.
    int64_t os[kMaxDims];
    int64_t acc = 1;
    for (int d = ndim - 1; d >= 0; --d) {
        os[d] = acc;
        acc *= shape[d];
    }
    MergedAxes m = merge_axes(shape, ndim, {a_strides, b_strides, os});
    if (m.empty) return MSST_OK;
    MSST_REQUIRE(a && b && out, MSST_ERR_INVALID_ARG, "null pointer");
    const size_t eb = dtype_bytes(dtype);
    MSST_REQUIRE(aligned(a, eb) && aligned(b, eb) && aligned(out, eb), MSST_ERR_ALIGNMENT,
                 "pointers must be aligned to the element size");
    const int in = m.ndim - 1;
    const int vec = (m.shape[in] % 4 == 0 && m.stride[0][in] <= 1 && m.stride[1][in] <= 1 &&
                     aligned(out, 4 * eb))
                        ? 4
                        : 1;
    if (vec == 4) m.shape[in] /= 4;
    IndexSpace sp;
    uint64_t total = 0;
    MSST_REQUIRE(make_index_space(m, sp, total), MSST_ERR_UNSUPPORTED,
                 "index space exceeds 2^62 elements");
    StrideSet as{}, bs{};
    for (int d = 0; d < m.ndim; ++d) {
        as.s[d] = m.stride[0][d];
        bs.s[d] = m.stride[1][d];
    }
    hipStream_t s = as_stream(stream);
    if (dtype == MSST_F16)
        launch_binary_op<half_t>(op, a, b, out, sp, as, bs, total, vec, s);
    else
        launch_binary_op<float>(op, a, b, out, sp, as, bs, total, vec, s);
    return check_launch("binary_kernel");
}
