// rope.hip — rotary position embedding.
//
// msst_rope_table builds the host table of model_bs_roformer.cu:205-230:
// freq_i = 1 / 10000^(2i/dh), angle = n * freq_i, evaluated in float exactly
// as the reference does, so any host evaluation and the GPU share one table.
//
// msst_rope_qk is the in-place ops::apply_rotary_emb (ops_misc.cu:39-131):
// interleaved pairs (2i, 2i+1) of q and k [B,H,N,D] rotate by the angle of
// (n, i).  f16 tensors are rotated in fp32 registers and rounded once (the
// reference's f16 path does the same through a f32 round trip).  One thread
// per pair; HBM-bound, 2 * 2 * B*H*N*D * elem bytes.
#include <math.h>

#include "msst_common.hpp"

namespace msst {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void rope_qk_kernel(T* __restrict__ q, T* __restrict__ k,
                                                      const float* __restrict__ cos_t,
                                                      const float* __restrict__ sin_t,
                                                      int64_t pairs, int N, int half) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= pairs) return;
    const int i = (int)(idx % half);
    const int n = (int)((idx / half) % N);
    const float c = cos_t[n * half + i], s = sin_t[n * half + i];
    T* qp = q + 2 * idx;
    T* kp = k + 2 * idx;
    float q0 = (float)qp[0], q1 = (float)qp[1];
    qp[0] = (T)(q0 * c - q1 * s);
    qp[1] = (T)(q0 * s + q1 * c);
    float k0 = (float)kp[0], k1 = (float)kp[1];
    kp[0] = (T)(k0 * c - k1 * s);
    kp[1] = (T)(k0 * s + k1 * c);
}

// Per-pair frequencies, computed on the host with the reference's float
// formula and passed by value, so the device angles (float)p * freq are
// bit-identical to the host table's; only cosf/sinf rounding may differ.
struct FreqTable {
    float v[64];
};

__global__ __launch_bounds__(256) void rope_table_kernel(int n, int half, FreqTable f,
                                                         float* __restrict__ cos_out,
                                                         float* __restrict__ sin_out) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= n * half) return;
    const int p = idx / half, i = idx % half;
    const float angle = (float)p * f.v[i];
    cos_out[idx] = cosf(angle);
    sin_out[idx] = sinf(angle);
}

}  // namespace
}  // namespace msst

extern "C" int msst_rope_table_device(int n, int dim_head, float* cos_out, float* sin_out,
                                      void* stream) {
    using namespace msst;
    MSST_REQUIRE(cos_out && sin_out, MSST_ERR_INVALID_ARG, "null output");
    MSST_REQUIRE(n >= 0 && dim_head > 0 && dim_head % 2 == 0, MSST_ERR_INVALID_ARG,
                 "dim_head must be positive and even");
    MSST_REQUIRE(dim_head <= 128, MSST_ERR_UNSUPPORTED, "dim_head must be <= 128");
    const int half = dim_head / 2;
    const int total = n * half;
    if (total == 0) return MSST_OK;
    FreqTable f{};
    for (int i = 0; i < half; ++i)
        f.v[i] = 1.0f / powf(10000.0f, (float)(2 * i) / (float)dim_head);
    hipLaunchKernelGGL(rope_table_kernel, dim3((total + 255) / 256), dim3(256), 0,
                       as_stream(stream), n, half, f, cos_out, sin_out);
    return check_launch("rope_table_kernel");
}

extern "C" int msst_rope_table(int n, int dim_head, float* cos_out, float* sin_out) {
    using namespace msst;
    MSST_REQUIRE(cos_out && sin_out, MSST_ERR_INVALID_ARG, "null output");
    MSST_REQUIRE(n >= 0 && dim_head > 0 && dim_head % 2 == 0, MSST_ERR_INVALID_ARG,
                 "dim_head must be positive and even");
    const int half = dim_head / 2;
    for (int p = 0; p < n; ++p)
        for (int i = 0; i < half; ++i) {
            float freq = 1.0f / powf(10000.0f, (float)(2 * i) / (float)dim_head);
            float angle = (float)p * freq;
            cos_out[p * half + i] = cosf(angle);
            sin_out[p * half + i] = sinf(angle);
        }
    return MSST_OK;
}

extern "C" int msst_rope_qk(void* q, void* k, int dtype, const float* cos_t, const float* sin_t,
                            int64_t B, int64_t H, int64_t N, int64_t D, void* stream) {
    using namespace msst;
    MSST_REQUIRE(q && k && cos_t && sin_t, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(B >= 0 && H >= 0 && N >= 0 && D > 0 && D % 2 == 0 && N < (1 << 30),
                 MSST_ERR_INVALID_ARG, "bad shape (D must be even)");
    MSST_REQUIRE(aligned(q, dtype_bytes(dtype)) && aligned(k, dtype_bytes(dtype)),
                 MSST_ERR_ALIGNMENT, "pointer not aligned to its element size");
    const int64_t pairs = B * H * N * (D / 2);
    if (pairs == 0) return MSST_OK;
    const unsigned grid = (unsigned)((pairs + 255) / 256);
    hipStream_t s = as_stream(stream);
    if (dtype == MSST_F16)
        hipLaunchKernelGGL(rope_qk_kernel<half_t>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<half_t*>(q), reinterpret_cast<half_t*>(k), cos_t,
                           sin_t, pairs, (int)N, (int)(D / 2));
    else
        hipLaunchKernelGGL(rope_qk_kernel<float>, dim3(grid), dim3(256), 0, s,
                           reinterpret_cast<float*>(q), reinterpret_cast<float*>(k), cos_t, sin_t,
                           pairs, (int)N, (int)(D / 2));
    return check_launch("rope_qk_kernel");
}
