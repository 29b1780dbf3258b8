// layout.hip — the layout and elementwise kernels the ops.h / Tensor layer
// needs around the hot path (all HBM-bound, vectorised where aligned):
//   msst_split_qkv_heads   [B,N,(3,H,D)] -> 3 x [B,H,N,D]
//                          (model_mel_band_roformer.cu:34-74, :117-140)
//   msst_gate_merge_heads  merged[b,n,h*D+d] = attn[b,h,n,d] * g[b,n,h]
//                          (model_mel_band_roformer.cu:76-115, :142-163)
//   msst_cast              f32 <-> f16 (tensor.cu:1269-1294)
//   msst_add               elementwise add (tensor.cu:1365-1447)
//   msst_tanh              elementwise tanh (ops_elementwise.cu:84-88, :138)
//   msst_complex_mul       product of interleaved complex pairs
//                          (ops_elementwise.cu:267-303)
//   msst_glu               last-axis GLU, first half * sigmoid(second half)
//                          (ops_elementwise.cu:321-388)
//   msst_chunk_extract     one chunk of the chunked driver: the audio seen
//                          through its border reflect padding, with the last
//                          chunk reflect- or zero-padded (inference_app.cpp:
//                          116-156)
//   msst_overlap_add       out += chunk * fade, weights += fade
//                          (ops_fused.cu:138-168; in stream order, no atomics)
//   msst_normalize_by_weights  out /= weights where > 1e-8 (ops_fused.cu:170-186)
//   msst_swap_axes12       [A,P,Q,R] -> [A,Q,P,R], the permute({0,2,1,3})
//                          .contiguous() of the depth loop
//                          (model_bs_roformer.cu:491, :509; tensor.cu:868-903)
// The fused Roformer stack does not use the first two: its attention kernel
// reads the packed qkv rows and writes merged, gated rows directly.
#include <algorithm>

#include "msst_common.hpp"

namespace msst {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void split_qkv_kernel(const T* __restrict__ qkv,
                                                        T* __restrict__ q, T* __restrict__ k,
                                                        T* __restrict__ v, int64_t total,
                                                        int64_t N, int64_t H, int64_t D) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    // idx enumerates [B,H,N,D] outputs.
    const int64_t d = idx % D;
    const int64_t n = (idx / D) % N;
    const int64_t h = (idx / (D * N)) % H;
    const int64_t b = idx / (D * N * H);
    const int64_t base = (b * N + n) * 3 * H * D + h * D + d;
    q[idx] = qkv[base];
    k[idx] = qkv[base + H * D];
    v[idx] = qkv[base + 2 * H * D];
}

template <typename T>
__global__ __launch_bounds__(256) void gate_merge_kernel(const T* __restrict__ attn,
                                                         const float* __restrict__ gates,
                                                         T* __restrict__ merged, int64_t total,
                                                         int64_t N, int64_t H, int64_t D) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    // idx enumerates merged [B,N,H,D] outputs (coalesced writes).
    const int64_t d = idx % D;
    const int64_t h = (idx / D) % H;
    const int64_t n = (idx / (D * H)) % N;
    const int64_t b = idx / (D * H * N);
    const float g = gates[(b * N + n) * H + h];
    merged[idx] = (T)((float)attn[((b * H + h) * N + n) * D + d] * g);
}

template <typename S, typename D>
__global__ __launch_bounds__(256) void cast_kernel(const S* __restrict__ src, D* __restrict__ dst,
                                                   int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) dst[i] = (D)(float)src[i];
}

// 4 elements per thread (n % 4 == 0, 16-byte aligned source).
template <typename S, typename D>
__global__ __launch_bounds__(256) void cast4_kernel(const S* __restrict__ src, D* __restrict__ dst,
                                                    int64_t n4) {
    typedef S SV __attribute__((ext_vector_type(4)));
    typedef D DV __attribute__((ext_vector_type(4)));
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n4; i += stride) {
        const SV v = reinterpret_cast<const SV*>(src)[i];
        reinterpret_cast<DV*>(dst)[i] = DV{(D)(float)v[0], (D)(float)v[1], (D)(float)v[2],
                                           (D)(float)v[3]};
    }
}

template <typename T>
__global__ __launch_bounds__(256) void add_kernel(const T* a, const T* b, T* out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) out[i] = (T)((float)a[i] + (float)b[i]);
}

template <typename T>
__global__ __launch_bounds__(256) void tanh_kernel(const T* x, T* out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) out[i] = (T)tanhf((float)x[i]);
}

// (a.re + i a.im)(b.re + i b.im) per interleaved complex pair.
__global__ __launch_bounds__(256) void complex_mul_kernel(const float2* __restrict__ a,
                                                          const float2* __restrict__ b,
                                                          float2* out, int64_t n) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const float2 x = a[i], y = b[i];
        out[i] = make_float2(x.x * y.x - x.y * y.y, x.x * y.y + x.y * y.x);
    }
}

// out[r, j] = x[r, j] * 1 / (1 + exp(-x[r, j + half])), x [rows, 2 half].
template <typename T>
__global__ __launch_bounds__(256) void glu_kernel(const T* __restrict__ x, T* __restrict__ out,
                                                  int64_t rows, int64_t half) {
    const int64_t n = rows * half;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const int64_t r = i / half, j = i - r * half;
        const float a = (float)x[r * 2 * half + j], g = (float)x[r * 2 * half + half + j];
        out[i] = (T)(a * (1.0f / (1.0f + expf(-g))));
    }
}

// Reflect index into [0, n) (edge sample not repeated; |p| < n).
__device__ __forceinline__ int64_t reflect_index(int64_t p, int64_t n) {
    if (p < 0) p = -p;
    if (p >= n) p = 2 * (n - 1) - p;
    return p;
}

// dst[c, i] for i < chunk: P[start + i] where P = audio reflect-padded by
// `border` on both sides; past the end of P, the chunk's own slice
// reflect-padded at its end (tail_reflect) or zero.
__global__ __launch_bounds__(256) void chunk_extract_kernel(const float* __restrict__ audio,
                                                            int64_t length, int64_t border,
                                                            int64_t start, int64_t chunk,
                                                            int tail_reflect,
                                                            float* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t c = blockIdx.y;
    if (i >= chunk) return;
    const int64_t plen = length + 2 * border;
    const int64_t actual = min(chunk, plen - start);
    float v = 0.0f;
    int64_t q = -1;
    if (i < actual)
        q = start + i;
    else if (tail_reflect)
        q = start + (2 * actual - 2 - i);
    if (q >= 0) v = audio[c * length + reflect_index(q - border, length)];
    dst[c * chunk + i] = v;
}

__global__ __launch_bounds__(256) void overlap_add_kernel(float* __restrict__ out,
                                                          float* __restrict__ wsum,
                                                          const float* __restrict__ src,
                                                          int64_t src_stride,
                                                          const float* __restrict__ window,
                                                          int64_t total, int64_t offset,
                                                          int64_t len) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t c = blockIdx.y;
    if (i >= len) return;
    const float w = window[i];
    out[c * total + offset + i] += src[c * src_stride + i] * w;
    if (c == 0) wsum[offset + i] += w;
}

__global__ __launch_bounds__(256) void normalize_by_weights_kernel(float* __restrict__ out,
                                                                   const float* __restrict__ wsum,
                                                                   int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t c = blockIdx.y;
    if (i >= total) return;
    const float w = wsum[i];
    if (w > 1e-8f) out[c * total + i] /= w;
}

// [A,P,Q,R] -> [A,Q,P,R]; one thread per 16-byte (or element) chunk of R.
template <typename V>
__global__ __launch_bounds__(256) void swap12_kernel(const V* __restrict__ src, V* __restrict__ dst,
                                                     int64_t A, int64_t P, int64_t Q, int64_t R) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int64_t stride = (int64_t)gridDim.x * blockDim.x;
    const int64_t total = A * P * Q * R;
    for (; idx < total; idx += stride) {
        // idx enumerates dst [A,Q,P,R] (coalesced writes)
        const int64_t r = idx % R;
        const int64_t pp = (idx / R) % P;
        const int64_t qq = (idx / (R * P)) % Q;
        const int64_t a = idx / (R * P * Q);
        dst[idx] = src[((a * P + pp) * Q + qq) * R + r];
    }
}

unsigned grid_for(int64_t n) {
    int64_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace
}  // namespace msst

extern "C" int msst_split_qkv_heads(const void* qkv, void* q, void* k, void* v, int dtype,
                                    int64_t B, int64_t N, int64_t H, int64_t D, void* stream) {
    using namespace msst;
    MSST_REQUIRE(qkv && q && k && v, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(B >= 0 && N >= 0 && H > 0 && D > 0, MSST_ERR_INVALID_ARG, "bad shape");
    const int64_t total = B * H * N * D;
    if (total == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(split_qkv_kernel<half_t>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(qkv), reinterpret_cast<half_t*>(q),
                           reinterpret_cast<half_t*>(k), reinterpret_cast<half_t*>(v), total, N,
                           H, D);
    else
        hipLaunchKernelGGL(split_qkv_kernel<float>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(qkv), reinterpret_cast<float*>(q),
                           reinterpret_cast<float*>(k), reinterpret_cast<float*>(v), total, N, H,
                           D);
    return check_launch("split_qkv_kernel");
}

extern "C" int msst_gate_merge_heads(const void* attn, const float* gates, void* merged,
                                     int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                                     void* stream) {
    using namespace msst;
    MSST_REQUIRE(attn && gates && merged, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(B >= 0 && N >= 0 && H > 0 && D > 0, MSST_ERR_INVALID_ARG, "bad shape");
    const int64_t total = B * H * N * D;
    if (total == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const unsigned grid = (unsigned)((total + 255) / 256);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(gate_merge_kernel<half_t>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(attn), gates,
                           reinterpret_cast<half_t*>(merged), total, N, H, D);
    else
        hipLaunchKernelGGL(gate_merge_kernel<float>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(attn), gates,
                           reinterpret_cast<float*>(merged), total, N, H, D);
    return check_launch("gate_merge_kernel");
}

extern "C" int msst_cast(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
                         void* stream) {
    using namespace msst;
    MSST_REQUIRE(src && dst, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(src_dtype) && is_dtype(dst_dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(n >= 0, MSST_ERR_INVALID_ARG, "negative size");
    if (n == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(n);
    if (n % 4 == 0 && aligned(src, 16) && aligned(dst, 16) && src_dtype != dst_dtype) {
        const unsigned g4 = grid_for(n / 4);
        if (src_dtype == MSST_F32)
            hipLaunchKernelGGL((cast4_kernel<float, half_t>), dim3(g4), dim3(256), 0, s,
                               reinterpret_cast<const float*>(src), reinterpret_cast<half_t*>(dst),
                               n / 4);
        else
            hipLaunchKernelGGL((cast4_kernel<half_t, float>), dim3(g4), dim3(256), 0, s,
                               reinterpret_cast<const half_t*>(src), reinterpret_cast<float*>(dst),
                               n / 4);
        return check_launch("cast4_kernel");
    }
    if (src_dtype == MSST_F32 && dst_dtype == MSST_F16)
        hipLaunchKernelGGL((cast_kernel<float, half_t>), dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(src), reinterpret_cast<half_t*>(dst), n);
    else if (src_dtype == MSST_F16 && dst_dtype == MSST_F32)
        hipLaunchKernelGGL((cast_kernel<half_t, float>), dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(src), reinterpret_cast<float*>(dst), n);
    else if (src_dtype == MSST_F32)
        hipLaunchKernelGGL((cast_kernel<float, float>), dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(src), reinterpret_cast<float*>(dst), n);
    else
        hipLaunchKernelGGL((cast_kernel<half_t, half_t>), dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(src), reinterpret_cast<half_t*>(dst), n);
    return check_launch("cast_kernel");
}

extern "C" int msst_add(const void* a, const void* b, void* out, int dtype, int64_t n,
                        void* stream) {
    using namespace msst;
    MSST_REQUIRE(a && b && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(n >= 0, MSST_ERR_INVALID_ARG, "negative size");
    if (n == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(n);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(add_kernel<half_t>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(a), reinterpret_cast<const half_t*>(b),
                           reinterpret_cast<half_t*>(out), n);
    else
        hipLaunchKernelGGL(add_kernel<float>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(a), reinterpret_cast<const float*>(b),
                           reinterpret_cast<float*>(out), n);
    return check_launch("add_kernel");
}

extern "C" int msst_complex_mul(const float* a, const float* b, float* out, int64_t n,
                                void* stream) {
    using namespace msst;
    MSST_REQUIRE(a && b && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(n >= 0, MSST_ERR_INVALID_ARG, "negative size");
    MSST_REQUIRE(aligned(a, 8) && aligned(b, 8) && aligned(out, 8), MSST_ERR_ALIGNMENT,
                 "complex pairs must be 8-byte aligned");
    if (n == 0) return MSST_OK;
    hipLaunchKernelGGL(complex_mul_kernel, dim3(grid_for(n)), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const float2*>(a), reinterpret_cast<const float2*>(b),
                       reinterpret_cast<float2*>(out), n);
    return check_launch("complex_mul_kernel");
}

extern "C" int msst_tanh(const void* x, void* out, int dtype, int64_t n, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(n >= 0, MSST_ERR_INVALID_ARG, "negative size");
    if (n == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(tanh_kernel<half_t>, dim3(grid_for(n)), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(x), reinterpret_cast<half_t*>(out), n);
    else
        hipLaunchKernelGGL(tanh_kernel<float>, dim3(grid_for(n)), dim3(256), 0, s,
                           reinterpret_cast<const float*>(x), reinterpret_cast<float*>(out), n);
    return check_launch("tanh_kernel");
}

extern "C" int msst_glu(const void* x, void* out, int dtype, int64_t rows, int64_t half,
                        void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && out && x != out, MSST_ERR_INVALID_ARG, "null or aliased tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(rows >= 0 && half >= 0, MSST_ERR_INVALID_ARG, "negative size");
    if (rows * half == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const unsigned grid = grid_for(rows * half);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(glu_kernel<half_t>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(x), reinterpret_cast<half_t*>(out),
                           rows, half);
    else
        hipLaunchKernelGGL(glu_kernel<float>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<const float*>(x), reinterpret_cast<float*>(out), rows,
                           half);
    return check_launch("glu_kernel");
}

extern "C" int msst_swap_axes12(const void* src, void* dst, int dtype, int64_t A, int64_t P,
                                int64_t Q, int64_t R, void* stream) {
    using namespace msst;
    MSST_REQUIRE(src && dst && src != dst, MSST_ERR_INVALID_ARG,
                 "null or aliased tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(A >= 0 && P >= 0 && Q >= 0 && R >= 0, MSST_ERR_INVALID_ARG, "bad shape");
    const int64_t total = A * P * Q * R;
    if (total == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const size_t rb = R * dtype_bytes(dtype);
    if (rb % 16 == 0 && aligned(src, 16) && aligned(dst, 16)) {
        const int64_t r16 = (int64_t)(rb / 16);
        hipLaunchKernelGGL(swap12_kernel<u4>, dim3(grid_for(A * P * Q * r16)), dim3(256), 0, s,
                           reinterpret_cast<const u4*>(src), reinterpret_cast<u4*>(dst), A, P, Q,
                           r16);
    } else if (dtype == MSST_F16) {
        hipLaunchKernelGGL(swap12_kernel<half_t>, dim3(grid_for(total)), dim3(256), 0, s,
                           reinterpret_cast<const half_t*>(src), reinterpret_cast<half_t*>(dst), A,
                           P, Q, R);
    } else {
        hipLaunchKernelGGL(swap12_kernel<float>, dim3(grid_for(total)), dim3(256), 0, s,
                           reinterpret_cast<const float*>(src), reinterpret_cast<float*>(dst), A, P,
                           Q, R);
    }
    return check_launch("swap12_kernel");
}

extern "C" int msst_chunk_extract(const float* audio, int64_t channels, int64_t length,
                                  int64_t border, int64_t start, int64_t chunk, int tail_reflect,
                                  float* dst, void* stream) {
    using namespace msst;
    MSST_REQUIRE(audio && dst, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(channels >= 1 && channels < 65536 && length >= 1 && chunk >= 1 && border >= 0,
                 MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(border < length, MSST_ERR_INVALID_ARG, "border reflect padding needs border < length");
    const int64_t plen = length + 2 * border;
    MSST_REQUIRE(start >= 0 && start < plen, MSST_ERR_INVALID_ARG, "chunk start out of range");
    const int64_t actual = std::min(chunk, plen - start);
    MSST_REQUIRE(!tail_reflect || actual == chunk || 2 * actual > chunk, MSST_ERR_INVALID_ARG,
                 "tail reflect padding needs more than half a chunk of signal");
    const dim3 grid((unsigned)((chunk + 255) / 256), (unsigned)channels);
    hipLaunchKernelGGL(chunk_extract_kernel, grid, dim3(256), 0, as_stream(stream), audio, length,
                       border, start, chunk, tail_reflect, dst);
    return check_launch("chunk_extract_kernel");
}

extern "C" int msst_overlap_add(float* out, float* wsum, const float* src, int64_t src_stride,
                                const float* window, int64_t channels, int64_t total,
                                int64_t offset, int64_t len, void* stream) {
    using namespace msst;
    MSST_REQUIRE(out && wsum && src && window, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(channels >= 1 && channels < 65536 && len >= 0 && offset >= 0 &&
                     offset + len <= total && src_stride >= len,
                 MSST_ERR_INVALID_ARG, "bad shape");
    if (len == 0) return MSST_OK;
    const dim3 grid((unsigned)((len + 255) / 256), (unsigned)channels);
    hipLaunchKernelGGL(overlap_add_kernel, grid, dim3(256), 0, as_stream(stream), out, wsum, src,
                       src_stride, window, total, offset, len);
    return check_launch("overlap_add_kernel");
}

extern "C" int msst_normalize_by_weights(float* out, const float* wsum, int64_t channels,
                                         int64_t total, void* stream) {
    using namespace msst;
    MSST_REQUIRE(out && wsum, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(channels >= 1 && channels < 65536 && total >= 0, MSST_ERR_INVALID_ARG,
                 "bad shape");
    if (total == 0) return MSST_OK;
    const dim3 grid((unsigned)((total + 255) / 256), (unsigned)channels);
    hipLaunchKernelGGL(normalize_by_weights_kernel, grid, dim3(256), 0, as_stream(stream), out,
                       wsum, total);
    return check_launch("normalize_by_weights_kernel");
}
