// gemm.hip — linear layers of the Roformer hot path on gfx950 MFMA.
//
//   out[M,N] = act(x[M,K] . W[N,K]^T + bias[N]) (+ residual[M,N])
//
// Replaces the cuBLAS GEMM + separate bias/activation kernels of
// ops_linear.cu:150-427 and ops_fused.cu:203-303, :341-358 with single
// kernels whose epilogue applies bias, activation and residual.
//
// Kernels
//   gemm_f16_kernel   f16 W (x f16 or f32, converted as it is staged):
//                     v_mfma_f32_32x32x16_f16, fp32 accumulation.
//   gemm_f32_kernel   f32 W: v_mfma_f32_32x32x2_f32 (true fp32, no TF32).
//   gemm_skinny       N <= 16 (the per-head gate projection): HBM-bound
//                     row dot products, one wave per row.
//   gemm_generic      any other shape (K not a multiple of the vector width).
//
// Tiling of the MFMA kernels: 256 threads = 4 waves in a 2x2 grid; each
// wave owns a (BM/2) x (BN/2) sub-tile held as 32x32 accumulator blocks.
// A and W tiles (BK along K) are staged through LDS in two buffers: the
// global loads for k-tile t+1 are issued before the MFMAs of tile t and
// written to the other buffer afterwards, so one barrier per k-tile
// suffices.  LDS rows are 128 bytes (8 chunks of 16 bytes); chunk c of row r
// is stored at c ^ (r & 7), which makes both the row-wise chunk stores and
// the 32-row fragment reads bank-conflict free.
//
// Tile order is XCD-aware: the hardware deals workgroups round-robin to the
// 8 XCDs, so workgroup b is given tile (b % 8) * per_xcd + b / 8 — every XCD
// walks a contiguous run of the row-major tile grid and the column tiles of
// a row block (which share the same A rows) run together in one L2.
#include "msst_common.hpp"

namespace msst {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ void tile_coords(int tiles_n, int per_xcd, int& tm, int& tn,
                                            int total) {
    int b = blockIdx.x;
    int t = (b & 7) * per_xcd + (b >> 3);
    if (t >= total) { tm = -1; tn = -1; return; }
    tm = t / tiles_n;
    tn = t - tm * tiles_n;
}

template <typename OutT>
__device__ __forceinline__ void epilogue_store(float v, int64_t row, int col, int N,
                                               const float* __restrict__ bias, int act,
                                               const OutT* residual, OutT* out) {
    if (bias) v += bias[col];
    v = act_apply(v, act);
    int64_t idx = row * (int64_t)N + col;
    if (residual) v += (float)residual[idx];
    out[idx] = (OutT)v;
}

// ---------------------------------------------------------------------------
// fp16 MFMA GEMM.  BK = 64 halves (one 128-byte LDS row per tile row).
// ---------------------------------------------------------------------------
template <int BM, int BN, bool A_F32, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_f16_kernel(
    const void* __restrict__ Aptr, const half_t* __restrict__ W,
    const float* __restrict__ bias, const OutT* residual, OutT* out,
    int M, int N, int K, int act, int tiles_n, int per_xcd) {
    constexpr int BK = 64;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_CH = BM * 8 / kThreads;  // 16-byte chunks per thread
    constexpr int B_CH = BN * 8 / kThreads;
    static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");

    __shared__ __attribute__((aligned(16))) half_t lds[2][(BM + BN) * BK];

    int tm, tn;
    tile_coords(tiles_n, per_xcd, tm, tn, ((M + BM - 1) / BM) * tiles_n);
    if (tm < 0) return;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;

    const int ld_row = tid >> 3;  // + 32*i
    const int ld_kc = tid & 7;

    h8 a_reg[A_CH];
    h8 b_reg[B_CH];

    auto load_tile = [&](int k0) {
        const int kk = k0 + ld_kc * 8;
        const bool kin = kk < K;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            int r = m0 + ld_row + 32 * i;
            if (kin && r < M) {
                if constexpr (A_F32) {
                    const float* src = reinterpret_cast<const float*>(Aptr) + (int64_t)r * K + kk;
                    f4 lo = *reinterpret_cast<const f4*>(src);
                    f4 hi = *reinterpret_cast<const f4*>(src + 4);
                    h8 v;
                    v[0] = (half_t)lo[0]; v[1] = (half_t)lo[1]; v[2] = (half_t)lo[2]; v[3] = (half_t)lo[3];
                    v[4] = (half_t)hi[0]; v[5] = (half_t)hi[1]; v[6] = (half_t)hi[2]; v[7] = (half_t)hi[3];
                    a_reg[i] = v;
                } else {
                    const half_t* src = reinterpret_cast<const half_t*>(Aptr) + (int64_t)r * K + kk;
                    a_reg[i] = *reinterpret_cast<const h8*>(src);
                }
            } else {
                a_reg[i] = h8{};
            }
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            int r = n0 + ld_row + 32 * i;
            if (kin && r < N)
                b_reg[i] = *reinterpret_cast<const h8*>(W + (int64_t)r * K + kk);
            else
                b_reg[i] = h8{};
        }
    };
    auto store_tile = [&](int buf) {
        half_t* As = lds[buf];
        half_t* Bs = lds[buf] + BM * BK;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            int r = ld_row + 32 * i;
            *reinterpret_cast<h8*>(As + r * BK + ((ld_kc ^ (r & 7)) << 3)) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            int r = ld_row + 32 * i;
            *reinterpret_cast<h8*>(Bs + r * BK + ((ld_kc ^ (r & 7)) << 3)) = b_reg[i];
        }
    };

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    const int KT = (K + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_tile((kt + 1) * BK);
        const half_t* As = lds[cur];
        const half_t* Bs = lds[cur] + BM * BK;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int c = kk * 2 + lhalf;
            h8 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                int r = wm * WM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const h8*>(As + r * BK + ((c ^ (r & 7)) << 3));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int r = wn * WN + j * 32 + lrow;
                bf[j] = *reinterpret_cast<const h8*>(Bs + r * BK + ((c ^ (r & 7)) << 3));
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) acc[i][j] = mfma32x32x16(af[i], bf[j], acc[i][j]);
        }
        if (kt + 1 < KT) store_tile(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int col = n0 + wn * WN + j * 32 + lrow;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * lhalf + (v & 3);
                if (row < M && col < N)
                    epilogue_store<OutT>(acc[i][j][v], row, col, N, bias, act, residual, out);
            }
        }
}

// ---------------------------------------------------------------------------
// fp32 MFMA GEMM.  BK = 32 floats (one 128-byte LDS row).  A lane of half h
// feeds K positions h*16 + s (s = 0..15) of each k-tile: four 16-byte LDS
// reads per operand fragment.
// ---------------------------------------------------------------------------
template <int BM, int BN, bool A_F16, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(
    const void* __restrict__ Aptr, const float* __restrict__ W,
    const float* __restrict__ bias, const OutT* residual, OutT* out,
    int M, int N, int K, int act, int tiles_n, int per_xcd) {
    constexpr int BK = 32;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_CH = BM * 8 / kThreads;
    constexpr int B_CH = BN * 8 / kThreads;

    __shared__ __attribute__((aligned(16))) float lds[2][(BM + BN) * BK];

    int tm, tn;
    tile_coords(tiles_n, per_xcd, tm, tn, ((M + BM - 1) / BM) * tiles_n);
    if (tm < 0) return;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int ld_row = tid >> 3;
    const int ld_kc = tid & 7;

    f4 a_reg[A_CH];
    f4 b_reg[B_CH];

    auto load_tile = [&](int k0) {
        const int kk = k0 + ld_kc * 4;
        const bool kin = kk < K;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            int r = m0 + ld_row + 32 * i;
            if (kin && r < M) {
                if constexpr (A_F16) {
                    h4 v = *reinterpret_cast<const h4*>(reinterpret_cast<const half_t*>(Aptr) +
                                                        (int64_t)r * K + kk);
                    a_reg[i] = f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
                } else {
                    a_reg[i] = *reinterpret_cast<const f4*>(reinterpret_cast<const float*>(Aptr) +
                                                            (int64_t)r * K + kk);
                }
            } else {
                a_reg[i] = f4{};
            }
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            int r = n0 + ld_row + 32 * i;
            if (kin && r < N)
                b_reg[i] = *reinterpret_cast<const f4*>(W + (int64_t)r * K + kk);
            else
                b_reg[i] = f4{};
        }
    };
    auto store_tile = [&](int buf) {
        float* As = lds[buf];
        float* Bs = lds[buf] + BM * BK;
#pragma unroll
        for (int i = 0; i < A_CH; ++i) {
            int r = ld_row + 32 * i;
            *reinterpret_cast<f4*>(As + r * BK + ((ld_kc ^ (r & 7)) << 2)) = a_reg[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; ++i) {
            int r = ld_row + 32 * i;
            *reinterpret_cast<f4*>(Bs + r * BK + ((ld_kc ^ (r & 7)) << 2)) = b_reg[i];
        }
    };

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    const int KT = (K + BK - 1) / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();

    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_tile((kt + 1) * BK);
        const float* As = lds[cur];
        const float* Bs = lds[cur] + BM * BK;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int c = lhalf * 4 + t;
            f4 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                int r = wm * WM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const f4*>(As + r * BK + ((c ^ (r & 7)) << 2));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int r = wn * WN + j * 32 + lrow;
                bf[j] = *reinterpret_cast<const f4*>(Bs + r * BK + ((c ^ (r & 7)) << 2));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = mfma32x32x2f32(af[i][s], bf[j][s], acc[i][j]);
        }
        if (kt + 1 < KT) store_tile(cur ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int col = n0 + wn * WN + j * 32 + lrow;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = m0 + wm * WM + i * 32 + 8 * (v >> 2) + 4 * lhalf + (v & 3);
                if (row < M && col < N)
                    epilogue_store<OutT>(acc[i][j][v], row, col, N, bias, act, residual, out);
            }
        }
}

// ---------------------------------------------------------------------------
// Skinny GEMM for N <= 16 (the H-wide gate projection): one wave per row,
// each lane a contiguous K slice, butterfly sums over the wave.
// ---------------------------------------------------------------------------
template <typename AT, typename WT, typename OutT, int NMAX>
__global__ __launch_bounds__(kThreads) void gemm_skinny_kernel(
    const AT* __restrict__ A, const WT* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int64_t M, int N, int K, int act) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * (kThreads / 64);
    for (int64_t row = wave; row < M; row += nwaves) {
        float acc[NMAX];
#pragma unroll
        for (int n = 0; n < NMAX; ++n) acc[n] = 0.0f;
        const AT* a = A + row * K;
        for (int k = lane; k < K; k += 64) {
            float av = (float)a[k];
#pragma unroll
            for (int n = 0; n < NMAX; ++n)
                if (n < N) acc[n] += av * (float)W[(int64_t)n * K + k];
        }
#pragma unroll
        for (int n = 0; n < NMAX; ++n) {
            if (n < N) {
                float s = wave_sum(acc[n]);
                if (lane == n) epilogue_store<OutT>(s, row, n, N, bias, act, residual, out);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Generic fallback: 16x16 output tile per 256-thread block, LDS-staged
// 16-wide K slices, fp32 accumulation.  Correct for any M, N, K and dtype.
// ---------------------------------------------------------------------------
template <typename AT, typename WT, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_generic_kernel(
    const AT* __restrict__ A, const WT* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int64_t M, int N, int K, int act) {
    __shared__ float As[16][17];
    __shared__ float Ws[16][17];
    const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const int64_t row = (int64_t)blockIdx.y * 16 + ty;
    const int col = blockIdx.x * 16 + tx;
    float acc = 0.0f;
    for (int k0 = 0; k0 < K; k0 += 16) {
        int64_t ar = (int64_t)blockIdx.y * 16 + ty;
        int wr = blockIdx.x * 16 + ty;
        As[ty][tx] = (ar < M && k0 + tx < K) ? (float)A[ar * K + k0 + tx] : 0.0f;
        Ws[ty][tx] = (wr < N && k0 + tx < K) ? (float)W[(int64_t)wr * K + k0 + tx] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; ++k) acc += As[ty][k] * Ws[tx][k];
        __syncthreads();
    }
    if (row < M && col < N) epilogue_store<OutT>(acc, row, col, N, bias, act, residual, out);
}

// ---------------------------------------------------------------------------
// Launch helpers.
// ---------------------------------------------------------------------------
int num_xcd_slots(int64_t tiles, int& per_xcd) {
    per_xcd = (int)((tiles + 7) / 8);
    return per_xcd * 8;
}

template <int BM, int BN, typename OutT>
int launch_f16(const void* x, bool x_f32, const half_t* w, const float* bias,
               const OutT* res, OutT* out, int M, int N, int K, int act, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int per_xcd;
    int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    if (x_f32)
        hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, true, OutT>), dim3(grid), dim3(kThreads), 0, s,
                           x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd);
    else
        hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, false, OutT>), dim3(grid), dim3(kThreads), 0, s,
                           x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd);
    return check_launch("gemm_f16_kernel");
}

template <int BM, int BN, typename OutT>
int launch_f32(const void* x, bool x_f16, const float* w, const float* bias,
               const OutT* res, OutT* out, int M, int N, int K, int act, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int per_xcd;
    int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    if (x_f16)
        hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, true, OutT>), dim3(grid), dim3(kThreads), 0, s,
                           x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, false, OutT>), dim3(grid), dim3(kThreads), 0, s,
                           x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd);
    return check_launch("gemm_f32_kernel");
}

template <typename AT, typename WT, typename OutT>
int launch_small(const void* x, const void* w, const float* bias, const OutT* res, OutT* out,
                 int64_t M, int N, int K, int act, hipStream_t s) {
    const AT* a = reinterpret_cast<const AT*>(x);
    const WT* wt = reinterpret_cast<const WT*>(w);
    if (N <= 16) {
        int64_t blocks = (M + 3) / 4;
        if (blocks > 8192) blocks = 8192;
        if (blocks < 1) blocks = 1;
        hipLaunchKernelGGL((gemm_skinny_kernel<AT, WT, OutT, 16>), dim3((unsigned)blocks),
                           dim3(kThreads), 0, s, a, wt, bias, res, out, M, N, K, act);
        return check_launch("gemm_skinny_kernel");
    }
    dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
    hipLaunchKernelGGL((gemm_generic_kernel<AT, WT, OutT>), grid, dim3(kThreads), 0, s, a, wt,
                       bias, res, out, M, N, K, act);
    return check_launch("gemm_generic_kernel");
}

template <typename OutT>
int dispatch(const void* x, int x_dtype, const void* w, int w_dtype, const float* bias,
             const void* residual, void* out, int64_t M, int64_t K, int64_t N, int act,
             hipStream_t s) {
    const OutT* res = reinterpret_cast<const OutT*>(residual);
    OutT* o = reinterpret_cast<OutT*>(out);
    const bool x_f32 = x_dtype == MSST_F32;
    const int m = (int)M, n = (int)N, k = (int)K;
    if (N <= 16 || M < 32) {
        if (w_dtype == MSST_F16)
            return x_f32 ? launch_small<float, half_t, OutT>(x, w, bias, res, o, M, n, k, act, s)
                         : launch_small<half_t, half_t, OutT>(x, w, bias, res, o, M, n, k, act, s);
        return x_f32 ? launch_small<float, float, OutT>(x, w, bias, res, o, M, n, k, act, s)
                     : launch_small<half_t, float, OutT>(x, w, bias, res, o, M, n, k, act, s);
    }
    if (w_dtype == MSST_F16) {
        const bool vec_ok = (K % 8 == 0) && aligned(x, 16) && aligned(w, 16);
        if (!vec_ok)
            return x_f32 ? launch_small<float, half_t, OutT>(x, w, bias, res, o, M, n, k, act, s)
                         : launch_small<half_t, half_t, OutT>(x, w, bias, res, o, M, n, k, act, s);
        if (N >= 1024)
            return launch_f16<256, 256, OutT>(x, x_f32, reinterpret_cast<const half_t*>(w), bias,
                                              res, o, m, n, k, act, s);
        return launch_f16<256, 128, OutT>(x, x_f32, reinterpret_cast<const half_t*>(w), bias, res,
                                          o, m, n, k, act, s);
    }
    const bool vec_ok = (K % 4 == 0) && aligned(x, x_f32 ? 16 : 8) && aligned(w, 16);
    if (!vec_ok)
        return x_f32 ? launch_small<float, float, OutT>(x, w, bias, res, o, M, n, k, act, s)
                     : launch_small<half_t, float, OutT>(x, w, bias, res, o, M, n, k, act, s);
    return launch_f32<128, 128, OutT>(x, !x_f32, reinterpret_cast<const float*>(w), bias, res, o,
                                      m, n, k, act, s);
}

}  // namespace
}  // namespace msst

extern "C" int msst_linear(const void* x, int x_dtype, const void* w, int w_dtype,
                           const float* bias, const void* residual, void* out, int out_dtype,
                           int64_t M, int64_t K, int64_t N, int act, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && w && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(x_dtype) && is_dtype(w_dtype) && is_dtype(out_dtype),
                 MSST_ERR_INVALID_ARG, "dtype must be MSST_F32 or MSST_F16");
    MSST_REQUIRE(M >= 0 && K > 0 && N > 0, MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(M < (int64_t)1 << 31 && K < (1 << 30) && N < (1 << 30), MSST_ERR_UNSUPPORTED,
                 "dimension exceeds 2^31");
    MSST_REQUIRE(act >= MSST_ACT_NONE && act <= MSST_ACT_SILU, MSST_ERR_INVALID_ARG,
                 "unknown activation");
    MSST_REQUIRE(aligned(x, dtype_bytes(x_dtype)) && aligned(w, dtype_bytes(w_dtype)) &&
                     aligned(out, dtype_bytes(out_dtype)) && aligned(bias, 4) &&
                     aligned(residual, dtype_bytes(out_dtype)),
                 MSST_ERR_ALIGNMENT, "pointer not aligned to its element size");
    if (M == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    if (out_dtype == MSST_F16)
        return dispatch<half_t>(x, x_dtype, w, w_dtype, bias, residual, out, M, K, N, act, s);
    return dispatch<float>(x, x_dtype, w, w_dtype, bias, residual, out, M, K, N, act, s);
}
