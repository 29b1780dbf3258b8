// norm.hip — RMSNorm of the Roformer layers, optionally fused with the
// per-head sigmoid gate projection that reads the same normalised row.
//
//   y = x * rsqrt(sum(x^2) + 1e-12) * gamma * scale        (ops_norm.cu:85-111)
//   gates[r, g] = sigmoid(y_r . w_gate[g] + b_gate[g])    (ops_fused.cu:285-303
//                                                          on the rms_norm output,
//                                                          model_bs_roformer.cu:268)
//
// One wave per row.  With D % 4 == 0 and D <= 1024 each lane holds up to
// four 4-element slots (elements 4*(64*i + lane) .. +3) in registers, so x
// is read once: 16-byte (f32) / 8-byte (f16) coalesced loads.  The sum of
// squares is a 6-step butterfly.  The G gate dot products are reduced with
// a reduce-scatter butterfly: the first shuffle halves the set of values a
// lane carries, so 8 gates cost 10 shuffles instead of 8 x 6.  Other D take
// a two-pass scalar path.  HBM-bound: bytes per row = D*(in + out) + 4G.
#include <type_traits>

#include "msst_common.hpp"

namespace msst {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;

template <typename T>
__device__ __forceinline__ f4 load4(const T* p);
template <>
__device__ __forceinline__ f4 load4<float>(const float* p) {
    return *reinterpret_cast<const f4*>(p);
}
template <>
__device__ __forceinline__ f4 load4<half_t>(const half_t* p) {
    h4 v = *reinterpret_cast<const h4*>(p);
    return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
template <typename T>
__device__ __forceinline__ void store4(T* p, f4 v);
template <>
__device__ __forceinline__ void store4<float>(float* p, f4 v) {
    *reinterpret_cast<f4*>(p) = v;
}
template <>
__device__ __forceinline__ void store4<half_t>(half_t* p, f4 v) {
    *reinterpret_cast<h4*>(p) = h4{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Reduce-scatter of GP (8 or 16) per-lane partial sums across the wave:
// afterwards lane l holds the full sum of value (l >> (6 - log2 GP)).
template <int GP>
__device__ __forceinline__ float reduce_scatter(float (&v)[GP], int lane) {
    constexpr int LOG = GP == 16 ? 4 : 3;
    float cur[GP];
#pragma unroll
    for (int i = 0; i < GP; ++i) cur[i] = v[i];
    int n = GP;
#pragma unroll
    for (int step = 0; step < LOG; ++step) {
        const int mask = 32 >> step;
        const bool upper = (lane & mask) != 0;
        n >>= 1;
#pragma unroll
        for (int i = 0; i < GP / 2; ++i) {
            if (i < n) {
                float send = upper ? cur[i] : cur[i + n];
                float keep = upper ? cur[i + n] : cur[i];
                cur[i] = keep + __shfl_xor(send, mask, 64);
            }
        }
    }
    float s = cur[0];
#pragma unroll
    for (int mask = 32 >> LOG; mask > 0; mask >>= 1) s += __shfl_xor(s, mask, 64);
    return s;
}

template <typename XT, typename OutT, typename WT, int GP>
__global__ __launch_bounds__(kThreads) void rms_norm_vec_kernel(
    const XT* __restrict__ x, const float* __restrict__ gamma, float scale,
    OutT* __restrict__ out, const WT* __restrict__ wg, const float* __restrict__ bg,
    float* __restrict__ gates, int64_t rows, int D, int G) {
    const int lane = threadIdx.x & 63;
    const int64_t wave0 = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
    for (int64_t row = wave0; row < rows; row += nwaves) {
        const XT* xr = x + row * D;
        f4 v[4];
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * (64 * i + lane);
            if (j < D) {
                v[i] = load4<XT>(xr + j);
                ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
            }
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss + 1e-12f);
        float gacc[GP > 0 ? GP : 1];
#pragma unroll
        for (int g = 0; g < (GP > 0 ? GP : 1); ++g) gacc[g] = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int j = 4 * (64 * i + lane);
            if (j < D) {
                f4 gm = *reinterpret_cast<const f4*>(gamma + j);
                f4 y;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // Rounded to the output type before the gate reads it,
                    // as the reference's linear_sigmoid reads the stored y.
                    y[e] = (float)(OutT)(v[i][e] * inv * gm[e] * scale);
                }
                store4<OutT>(out + row * D + j, y);
                if constexpr (GP > 0) {
#pragma unroll
                    for (int g = 0; g < GP; ++g) {
                        if (g < G) {
                            f4 w = load4<WT>(wg + (int64_t)g * D + j);
                            gacc[g] += y[0] * w[0] + y[1] * w[1] + y[2] * w[2] + y[3] * w[3];
                        }
                    }
                }
            }
        }
        if constexpr (GP > 0) {
            float s = reduce_scatter<GP>(gacc, lane);
            constexpr int SHIFT = GP == 16 ? 2 : 3;
            const int g = lane >> SHIFT;
            if ((lane & ((1 << SHIFT) - 1)) == 0 && g < G)
                gates[row * G + g] = sigmoid_fast(s + bg[g]);
        }
    }
}

// fp16 output and fp16 gate weights (the Roformer fp16 path): each wave
// walks a grid-stride run of rows and keeps its slice of gamma and of
// W_gate [G, D] in registers for the whole run (NS slots of 4 columns per
// lane, D <= 256 * NS), so W_gate is read once per wave instead of once per
// row.  The gate dot products run on the fp16-rounded y with v_dot2_f32_f16
// (fp32 accumulation of exact fp16 products, as a GEMM over the stored y
// computes them).  The next row's x is loaded before the current row is
// processed.
template <typename XT, int NS, int GP>
__global__ __launch_bounds__(kThreads) void rms_norm_gate_h_kernel(
    const XT* __restrict__ x, const float* __restrict__ gamma, float scale,
    half_t* __restrict__ out, const half_t* __restrict__ wg, const float* __restrict__ bg,
    float* __restrict__ gates, int64_t rows, int D, int G) {
    const int lane = threadIdx.x & 63;
    // Wave-uniform (readfirstlane), so the per-row buffer resources stay in SGPRs.
    const int64_t wave0 =
        (int64_t)blockIdx.x * kRowsPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
    if (wave0 >= rows) return;
    f4 gm[NS];
    h2 wr[NS][GP][2];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int j = 4 * (64 * i + lane);
        const bool in = j < D;
        gm[i] = in ? *reinterpret_cast<const f4*>(gamma + j) : f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int g = 0; g < GP; ++g) {
            h4 w = h4{};
            if (in && g < G) w = *reinterpret_cast<const h4*>(wg + (int64_t)g * D + j);
            wr[i][g][0] = h2{w[0], w[1]};
            wr[i][g][1] = h2{w[2], w[3]};
        }
    }
    // Every global access goes through a per-row buffer resource: rows past
    // the end and columns past D read zero / drop their stores in hardware,
    // so the loop has no data-dependent branch and the compiler's waits
    // cover only the data each step needs (with branches it waited for the
    // prefetched row right after issuing it).  Cross-lane sums use DPP moves
    // (dpp_wave_sum): the gate sums of all G heads end wave-uniform, and
    // lane g < G finishes and stores gate g.
    const uint32_t kDrop = 0x80000000u;
    uint32_t xoff[NS], ooff[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int j = 4 * (64 * i + lane);
        xoff[i] = j < D ? (uint32_t)(j * (int)sizeof(XT)) : kDrop;
        ooff[i] = j < D ? (uint32_t)(j * 2) : kDrop;
    }
    // GP == 8: gate g is finished in lanes 8g .. 8g + 7 and stored by lane 8g.
    const int gl = GP == 8 ? lane >> 3 : lane;
    const bool gstore = GP == 8 ? ((lane & 7) == 0 && gl < G) : lane < G;
    const float bgl = gl < G ? bg[gl] : 0.0f;
    const uint32_t goff = gstore ? (uint32_t)(gl * 4) : kDrop;
    auto load_row = [&](int64_t r, f4 (&dst)[NS]) {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<XT*>(x) + (r < rows ? r : 0) * D, (short)0,
            r < rows ? D * (int)sizeof(XT) : 0, 0x00020000);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            if constexpr (std::is_same<XT, float>::value) {
                dst[i] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, xoff[i], 0, 0));
            } else {
                const h4 hv = __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(rs, xoff[i], 0, 0));
                dst[i] = f4{(float)hv[0], (float)hv[1], (float)hv[2], (float)hv[3]};
            }
        }
    };
    auto process = [&](int64_t row, const f4 (&v)[NS]) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < NS; ++i)
            ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        const float inv = 1.0f / sqrtf(dpp_wave_sum(ss) + 1e-12f);
        float gacc[GP];
#pragma unroll
        for (int g = 0; g < GP; ++g) gacc[g] = 0.0f;
        const bool live = row < rows;  // a row past the end computes on zeros, stores nothing
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            out + (live ? row : 0) * D, (short)0, live ? D * 2 : 0, 0x00020000);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            h4 y;
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = (half_t)(v[i][e] * inv * gm[i][e] * scale);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, y), ro, ooff[i], 0, 0);
            const h2 y0 = h2{y[0], y[1]}, y1 = h2{y[2], y[3]};
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                gacc[g] = __builtin_amdgcn_fdot2(y0, wr[i][g][0], gacc[g], false);
                gacc[g] = __builtin_amdgcn_fdot2(y1, wr[i][g][1], gacc[g], false);
            }
        }
        float mine = 0.0f;
        if constexpr (GP == 8) {
            mine = gate_sums8(gacc, lane);
        } else {
#pragma unroll
            for (int g = 0; g < GP; ++g) {
                const float tot = dpp_wave_sum(gacc[g]);
                mine = lane == g ? tot : mine;
            }
        }
        const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
            gates + (live ? row : 0) * G, (short)0, live ? G * 4 : 0, 0x00020000);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sigmoid_fast(mine + bgl)),
                                              rg, goff, 0, 0);
    };
    // Two row buffers in turn: one row is processed while the next loads.
    // Both halves run unconditionally (the second may be a row past the
    // end): a branch between them lets the compiler sink the load of the
    // second row next to its use.  The scheduling fences keep each load
    // ahead of the other row's work.
    f4 va[NS], vb[NS];
    load_row(wave0, va);
    for (int64_t row = wave0; row < rows; row += 2 * nwaves) {
        load_row(row + nwaves, vb);
        __builtin_amdgcn_sched_barrier(0);
        process(row, va);
        load_row(row + 2 * nwaves, va);
        __builtin_amdgcn_sched_barrier(0);
        process(row + nwaves, vb);
    }
}

template <typename XT, int NS, int GP>
void launch_gate_h(const void* x, const float* gamma, float scale, void* out, const void* wg,
                   const float* bg, float* gates, int64_t rows, int D, int G, hipStream_t s) {
    // At most 4096 waves, each with the same number of rows (a wave striding
    // by the wave count would otherwise leave the last row-time to a few).
    const int64_t per_wave = (rows + 4095) / 4096;
    const int64_t nw = (rows + per_wave - 1) / per_wave;
    const int64_t blocks = (nw + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL((rms_norm_gate_h_kernel<XT, NS, GP>), dim3((unsigned)blocks),
                       dim3(kThreads), 0, s, reinterpret_cast<const XT*>(x), gamma, scale,
                       reinterpret_cast<half_t*>(out), reinterpret_cast<const half_t*>(wg), bg,
                       gates, rows, D, G);
}

// Any D: two passes over the row, scalar accesses.
template <typename XT, typename OutT, typename WT, int GP>
__global__ __launch_bounds__(kThreads) void rms_norm_scalar_kernel(
    const XT* __restrict__ x, const float* __restrict__ gamma, float scale,
    OutT* __restrict__ out, const WT* __restrict__ wg, const float* __restrict__ bg,
    float* __restrict__ gates, int64_t rows, int D, int G) {
    const int lane = threadIdx.x & 63;
    const int64_t wave0 = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * kRowsPerBlock;
    for (int64_t row = wave0; row < rows; row += nwaves) {
        const XT* xr = x + row * D;
        float ss = 0.0f;
        for (int j = lane; j < D; j += 64) {
            float a = (float)xr[j];
            ss += a * a;
        }
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss + 1e-12f);
        float gacc[GP > 0 ? GP : 1];
#pragma unroll
        for (int g = 0; g < (GP > 0 ? GP : 1); ++g) gacc[g] = 0.0f;
        for (int j = lane; j < D; j += 64) {
            float y = (float)(OutT)((float)xr[j] * inv * gamma[j] * scale);
            out[row * D + j] = (OutT)y;
            if constexpr (GP > 0) {
#pragma unroll
                for (int g = 0; g < GP; ++g)
                    if (g < G) gacc[g] += y * (float)wg[(int64_t)g * D + j];
            }
        }
        if constexpr (GP > 0) {
            float s = reduce_scatter<GP>(gacc, lane);
            constexpr int SHIFT = GP == 16 ? 2 : 3;
            const int g = lane >> SHIFT;
            if ((lane & ((1 << SHIFT) - 1)) == 0 && g < G)
                gates[row * G + g] = sigmoid_fast(s + bg[g]);
        }
    }
}

template <typename XT, typename OutT, typename WT, int GP>
int launch_norm(const void* x, const float* gamma, float scale, void* out, const void* wg,
                const float* bg, float* gates, int64_t rows, int D, int G, hipStream_t s) {
    int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    if (blocks > 16384) blocks = 16384;
    const bool vec = (D % 4 == 0) && D <= 1024 && aligned(x, 4 * sizeof(XT)) &&
                     aligned(out, 4 * sizeof(OutT)) && aligned(gamma, 16) &&
                     (GP == 0 || aligned(wg, 4 * sizeof(WT)));
    if (vec)
        hipLaunchKernelGGL((rms_norm_vec_kernel<XT, OutT, WT, GP>), dim3((unsigned)blocks),
                           dim3(kThreads), 0, s, reinterpret_cast<const XT*>(x), gamma, scale,
                           reinterpret_cast<OutT*>(out), reinterpret_cast<const WT*>(wg), bg,
                           gates, rows, D, G);
    else
        hipLaunchKernelGGL((rms_norm_scalar_kernel<XT, OutT, WT, GP>), dim3((unsigned)blocks),
                           dim3(kThreads), 0, s, reinterpret_cast<const XT*>(x), gamma, scale,
                           reinterpret_cast<OutT*>(out), reinterpret_cast<const WT*>(wg), bg,
                           gates, rows, D, G);
    return check_launch("rms_norm kernel");
}

template <typename XT, typename OutT>
int dispatch_gate(const void* x, const float* gamma, float scale, void* out, const void* wg,
                  int w_dtype, const float* bg, float* gates, int64_t rows, int D, int G,
                  hipStream_t s) {
    if (G == 0)
        return launch_norm<XT, OutT, float, 0>(x, gamma, scale, out, nullptr, nullptr, nullptr,
                                               rows, D, 0, s);
    if constexpr (std::is_same<OutT, half_t>::value) {
        // Register-resident W_gate path: D % 4 == 0, D <= 1024, aligned rows.
        const bool fast = w_dtype == MSST_F16 && D % 4 == 0 && D <= 1024 &&
                          aligned(x, 4 * sizeof(XT)) && aligned(out, 8) && aligned(gamma, 16) &&
                          aligned(wg, 8);
        if (fast) {
            const int ns = (D + 255) / 256;
            if (G <= 8) {
                if (ns == 1) launch_gate_h<XT, 1, 8>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else if (ns == 2) launch_gate_h<XT, 2, 8>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else if (ns == 3) launch_gate_h<XT, 3, 8>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else launch_gate_h<XT, 4, 8>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
            } else {
                if (ns == 1) launch_gate_h<XT, 1, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else if (ns == 2) launch_gate_h<XT, 2, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else if (ns == 3) launch_gate_h<XT, 3, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
                else launch_gate_h<XT, 4, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
            }
            return check_launch("rms_norm_gate_h_kernel");
        }
    }
    if (w_dtype == MSST_F16) {
        if (G <= 8)
            return launch_norm<XT, OutT, half_t, 8>(x, gamma, scale, out, wg, bg, gates, rows, D,
                                                    G, s);
        return launch_norm<XT, OutT, half_t, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G,
                                                 s);
    }
    if (G <= 8)
        return launch_norm<XT, OutT, float, 8>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
    return launch_norm<XT, OutT, float, 16>(x, gamma, scale, out, wg, bg, gates, rows, D, G, s);
}

int norm_common(const void* x, int x_dtype, const float* gamma, float scale, void* out,
                int out_dtype, const void* wg, int w_dtype, const float* bg, float* gates,
                int64_t rows, int64_t D, int G, void* stream) {
    hipStream_t s = as_stream(stream);
    const int d = (int)D;
    if (x_dtype == MSST_F32) {
        if (out_dtype == MSST_F32)
            return dispatch_gate<float, float>(x, gamma, scale, out, wg, w_dtype, bg, gates, rows,
                                               d, G, s);
        return dispatch_gate<float, half_t>(x, gamma, scale, out, wg, w_dtype, bg, gates, rows, d,
                                            G, s);
    }
    if (out_dtype == MSST_F32)
        return dispatch_gate<half_t, float>(x, gamma, scale, out, wg, w_dtype, bg, gates, rows, d,
                                            G, s);
    return dispatch_gate<half_t, half_t>(x, gamma, scale, out, wg, w_dtype, bg, gates, rows, d, G,
                                         s);
}

}  // namespace
}  // namespace msst

extern "C" int msst_rms_norm(const void* x, int x_dtype, const float* gamma, float scale,
                             void* out, int out_dtype, int64_t rows, int64_t D, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && gamma && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(x_dtype) && is_dtype(out_dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(rows >= 0 && D > 0 && D < (1 << 30), MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(aligned(x, dtype_bytes(x_dtype)) && aligned(out, dtype_bytes(out_dtype)) &&
                     aligned(gamma, 4),
                 MSST_ERR_ALIGNMENT, "pointer not aligned to its element size");
    if (rows == 0) return MSST_OK;
    return norm_common(x, x_dtype, gamma, scale, out, out_dtype, nullptr, MSST_F32, nullptr,
                       nullptr, rows, D, 0, stream);
}

extern "C" int msst_rms_norm_gate(const void* x, int x_dtype, const float* gamma, float scale,
                                  void* out, int out_dtype, const void* w_gate, int w_dtype,
                                  const float* b_gate, float* gates, int64_t rows, int64_t D,
                                  int G, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && gamma && out && w_gate && b_gate && gates, MSST_ERR_INVALID_ARG,
                 "null tensor pointer");
    MSST_REQUIRE(is_dtype(x_dtype) && is_dtype(out_dtype) && is_dtype(w_dtype),
                 MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(rows >= 0 && D > 0 && D < (1 << 30), MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(G >= 1 && G <= 16, MSST_ERR_UNSUPPORTED, "gate count must be 1..16");
    MSST_REQUIRE(aligned(x, dtype_bytes(x_dtype)) && aligned(out, dtype_bytes(out_dtype)) &&
                     aligned(gamma, 4) && aligned(w_gate, dtype_bytes(w_dtype)) &&
                     aligned(b_gate, 4) && aligned(gates, 4),
                 MSST_ERR_ALIGNMENT, "pointer not aligned to its element size");
    if (rows == 0) return MSST_OK;
    return norm_common(x, x_dtype, gamma, scale, out, out_dtype, w_gate, w_dtype, b_gate, gates,
                       rows, D, G, stream);
}
