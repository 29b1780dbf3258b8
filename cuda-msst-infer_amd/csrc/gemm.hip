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
//   gemm_f32_dma_kernel / gemm_f32_kernel
//                     f32 W: v_mfma_f32_32x32x2_f32 (true fp32, no TF32); f32 x
//                     with K % 32 == 0 through LDS DMA, otherwise staged.
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
#include <algorithm>
#include <type_traits>

#include "epilogue.hpp"
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
template <int BM, int BN, bool A_F32, bool RES, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_f16_kernel(
    const void* __restrict__ Aptr, const half_t* __restrict__ W,
    const float* __restrict__ bias, const OutT* residual, OutT* out,
    int M, int N, int K, int act, int tiles_n, int per_xcd, int vec) {
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

    constexpr int kRegion = (int)(sizeof(lds) / sizeof(float) / 4);
    constexpr int kIP = pick_ip<MI, WN, kRegion>();
    static_assert(kIP * 32 * WN <= kRegion, "epilogue staging does not fit in LDS");
    store_tile_lds<MI, NI, kIP, RES ? kEpiRes : kEpiPlain, OutT>(acc, reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion,
                                      lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act, residual,
                                      out, vec != 0);
}

// ---------------------------------------------------------------------------
// fp32 MFMA GEMM.  BK = 32 floats (one 128-byte LDS row).  A lane of half h
// feeds K positions h*16 + s (s = 0..15) of each k-tile: four 16-byte LDS
// reads per operand fragment.
// ---------------------------------------------------------------------------
template <int BM, int BN, bool A_F16, bool RES, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(
    const void* __restrict__ Aptr, const float* __restrict__ W,
    const float* __restrict__ bias, const OutT* residual, OutT* out,
    int M, int N, int K, int act, int tiles_n, int per_xcd, int vec) {
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

    constexpr int kRegion = (int)(sizeof(lds) / sizeof(float) / 4);
    constexpr int kIP = pick_ip<MI, WN, kRegion>();
    static_assert(kIP * 32 * WN <= kRegion, "epilogue staging does not fit in LDS");
    store_tile_lds<MI, NI, kIP, RES ? kEpiRes : kEpiPlain, OutT>(acc, reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion,
                                      lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act, residual,
                                      out, vec != 0);
}

// ---------------------------------------------------------------------------
// fp32 x and W through LDS DMA (K % 32 == 0, 16-byte aligned rows, each
// operand under 2 GiB): the tile and fragment reads of gemm_f32_kernel,
// without staging every k-tile through VGPRs and ds_write.  A
// buffer_load_dwordx4 ... lds writes 64 lanes x 16 bytes of LDS rows; lane
// l fetches the source chunk that the row's XOR swizzle puts at its
// position, so the fragment reads need no other change.  Rows past M / N
// are clamped to the last valid row (their results are never stored).  Two
// stages: the DMA of k-tile t + 1 is issued right after the barrier that
// opens k-tile t, one k-tile of MFMAs ahead of its use.
// BK = 32 (64 KB of LDS, two workgroups per CU) would keep the MFMA order
// of gemm_f32_kernel and so its bits.  BK = 16 (32 KB) lets four workgroups
// share a CU: 54 VGPRs, and 53 for the residual epilogue with 2 rows per
// batch (143 with 8).  fp32 MelBandRoformer layer against BK = 32: QKV
// 494 -> 467 us, FF1 472 -> 442, out-projection 190 -> 172, FF2 475 -> 450;
// the K pairs summed per MFMA differ, so the last bits do.
// ---------------------------------------------------------------------------
template <int BM, int BN, int BK, bool RES, typename OutT>
__global__ __launch_bounds__(kThreads) void gemm_f32_dma_kernel(
    const float* __restrict__ A, const float* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int M, int N, int K, int act, int tiles_n, int per_xcd,
    int vec) {
    static_assert(BK == 32 || BK == 16, "k-tile of 32 or 16 floats");
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int CPR = BK / 4;               // 16-byte chunks per LDS row
    constexpr int RPI = 64 / CPR;             // LDS rows per DMA instruction
    constexpr int NWAVE = kThreads / 64;
    constexpr int A_INST = BM / RPI / NWAVE;  // per wave and k-tile
    constexpr int B_INST = BN / RPI / NWAVE;
    static_assert(A_INST * RPI * NWAVE == BM && B_INST * RPI * NWAVE == BN, "DMA split");

    __shared__ __attribute__((aligned(16))) float lds[2][(BM + BN) * BK];

    int tm, tn;
    tile_coords(tiles_n, per_xcd, tm, tn, ((M + BM - 1) / BM) * tiles_n);
    if (tm < 0) return;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wid >> 1, wn = wid & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int sub = lane / CPR, pch = lane % CPR;
    // Chunk c of LDS row r sits at c ^ swz(r): 128-byte rows rotate by r, 64-byte rows by
    // r / 4, so the 16 rows one b128 read pass touches fall in distinct banks.
    auto swz = [](int r) { return CPR == 8 ? (r & 7) : ((r >> 2) & 3); };

    const int a_bytes = M * K * 4, b_bytes = N * K * 4;  // < 2^31 (checked on the host)
    uint32_t aoff[A_INST], boff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int rl = (wid * A_INST + i) * RPI + sub;
        aoff[i] = (uint32_t)(min(m0 + rl, M - 1) * K + ((pch ^ swz(rl)) << 2)) * 4u;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int rl = (wid * B_INST + i) * RPI + sub;
        boff[i] = (uint32_t)(min(n0 + rl, N - 1) * K + ((pch ^ swz(rl)) << 2)) * 4u;
    }
    auto issue = [&](int kt, int buf) {
        const uint32_t kb = (uint32_t)(kt * BK) * 4u;
        half_t* base = reinterpret_cast<half_t*>(&lds[buf][0]);  // 1 KB = 512 halves per DMA
#pragma unroll
        for (int i = 0; i < A_INST; ++i) dma16(A, a_bytes, base + (wid * A_INST + i) * 512, aoff[i] + kb);
#pragma unroll
        for (int i = 0; i < B_INST; ++i)
            dma16(W, b_bytes, base + BM * BK * 2 + (wid * B_INST + i) * 512, boff[i] + kb);
    };

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    const int KT = K / BK;
    issue(0, 0);
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        // k-tile kt has landed for this wave; after the barrier, for every
        // wave, and every wave has finished reading buffer cur ^ 1 (k-tile
        // kt - 1), which the next DMA overwrites.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (kt + 1 < KT) issue(kt + 1, cur ^ 1);
        const float* As = lds[cur];
        const float* Bs = lds[cur] + BM * BK;
#pragma unroll
        for (int t = 0; t < BK / 8; ++t) {
            const int c = lhalf * (BK / 8) + t;
            f4 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                int r = wm * WM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const f4*>(As + r * BK + ((c ^ swz(r)) << 2));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                int r = wn * WN + j * 32 + lrow;
                bf[j] = *reinterpret_cast<const f4*>(Bs + r * BK + ((c ^ swz(r)) << 2));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int j = 0; j < NI; ++j)
                        acc[i][j] = mfma32x32x2f32(af[i][s], bf[j][s], acc[i][j]);
        }
    }
    lds_barrier();  // every wave is done with the last k-tile before the epilogue reuses LDS

    constexpr int kRegion = (int)(sizeof(lds) / sizeof(float) / 4);
    constexpr int kIP = pick_ip<MI, WN, kRegion>();
    static_assert(kIP * 32 * WN <= kRegion, "epilogue staging does not fit in LDS");
    store_tile_lds<MI, NI, kIP, RES ? kEpiRes : kEpiPlain, OutT, false, -1, false, false, RES ? 2 : 8>(acc, reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion,
                                      lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act, residual,
                                      out, vec != 0);
}

// ---------------------------------------------------------------------------
// fp16 MFMA GEMM fed by LDS DMA (the fast path: f16 x, f16 W, K % 64 == 0).
//
// Tiles move global -> LDS with buffer_load_dwordx4 ... lds: each
// instruction writes 64 lanes x 16 bytes = 8 tile rows of 128 bytes
// contiguously, so the XOR swizzle is applied on the source side (lane l
// fetches logical chunk (l & 7) ^ (l >> 3) of row l >> 3).  No VGPRs stage
// the tiles and no ds_write is issued.  Rows past M / N are clamped to the
// last valid row (their results are never stored).  The next k-tile's DMA
// is issued before the current tile's MFMAs; fragments of k-substep kk+1
// are read from LDS while the MFMAs of kk run.  One vmcnt wait + barrier
// per k-tile.
// ---------------------------------------------------------------------------
template <int BK>
__device__ __forceinline__ int chunk_swz(int r) {
    // LDS rows of BK halves = BK/8 chunks of 16 B.  A b128 read is serviced
    // 16 lanes (256 bytes, 64 banks) at a time; the 16 lanes read the same
    // logical chunk of 16 consecutive rows, so the XOR must give those rows
    // 16 distinct 16-byte bank groups: (r >> 1) & 7 for 128-byte rows (odd
    // rows already sit 32 banks over), (r >> 2) & 3 for 64-byte rows.
    if constexpr (BK == 64) return ((r >> 1) & 7);
    else return ((r >> 2) & 3);
}

// BK = 64 (128-byte LDS rows) or 32 (64-byte rows).  NSTG = LDS ring
// stages: the prologue fills the whole ring, and the DMA of k-tile t + NSTG
// is issued as soon as every wave has finished reading tile t's slot (in
// the middle of k-tile t), so a load has about NSTG - 1 k-tiles of MFMA time
// to land.  The per-k-tile barrier is fence-free (lds_barrier):
// __syncthreads() would add s_waitcnt vmcnt(0) and wait for the younger
// stages too, serialising the ring.  MINB = workgroups per CU the register/LDS budget is sized for
// (3 for 128x128 tiles, so one workgroup's prologue and epilogue latency
// overlaps the others' main loops; 1 for the 8-wave 256x256 tile).  NWN =
// waves along N (2 x NWN waves, each owning a (BM/2) x (BN/NWN) sub-tile).
template <int BM, int BN, int BK, int NSTG, int MINB, int NWN, int EPI, int ACT, typename OutT>
__global__ __launch_bounds__(128 * NWN, MINB) void gemm_f16_dma_kernel(
    const half_t* __restrict__ A, const half_t* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int M, int N, int K, int act, int tiles_n, int per_xcd,
    int vec, EpiRope rope) {
    constexpr int CPR = BK / 8;              // 16-byte chunks per LDS row
    constexpr int RPD = 64 / CPR;            // rows per 1 KB DMA instruction
    constexpr int KK = BK / 16;              // MFMA k-substeps per k-tile
    constexpr int NW = 2 * NWN;              // waves: 2 along M x NWN along N
    constexpr int WM = BM / 2, WN = BN / NWN;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_INST = BM / RPD / NW;    // DMA instructions per wave per k-tile
    constexpr int B_INST = BN / RPD / NW;
    static_assert(A_INST * RPD * NW == BM && B_INST * RPD * NW == BN, "DMA split");
    constexpr int STAGE = (BM + BN) * BK;    // halves per LDS buffer
    static_assert(A_INST >= 1 && B_INST >= 1, "tile too small for the DMA split");
    static_assert(NSTG >= 2 && (NSTG - 1) * (A_INST + B_INST) <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(16))) half_t lds[NSTG][STAGE];

    int tm, tn;
    tile_coords(tiles_n, per_xcd, tm, tn, ((M + BM - 1) / BM) * tiles_n);
    if (tm < 0) return;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wid = tid >> 6;
    const int wm = wid / NWN, wn = wid % NWN;
    const int lrow = lane & 31, lhalf = lane >> 5;

    const int a_bytes = M * K * 2, b_bytes = N * K * 2;
    const int sub_row = lane / CPR;
    uint32_t aoff[A_INST], boff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int rl = (wid * A_INST + i) * RPD + sub_row;  // row within the tile
        const int lchunk = (lane % CPR) ^ chunk_swz<BK>(rl);
        const int r = min(m0 + rl, M - 1);
        aoff[i] = (uint32_t)(r * K + lchunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int rl = (wid * B_INST + i) * RPD + sub_row;
        const int lchunk = (lane % CPR) ^ chunk_swz<BK>(rl);
        const int r = min(n0 + rl, N - 1);
        boff[i] = (uint32_t)(r * K + lchunk * 8) * 2u;
    }
    // DMA instruction `idx` (0 .. A_INST+B_INST-1) of the k-tile at k0.
    auto issue_one = [&](int idx, int k0, int buf) {
        const uint32_t kb = (uint32_t)k0 * 2u;
        if (idx < A_INST)
            dma16(A, a_bytes, lds[buf] + (wid * A_INST + idx) * 512, aoff[idx] + kb);
        else
            dma16(W, b_bytes, lds[buf] + BM * BK + (wid * B_INST + idx - A_INST) * 512,
                  boff[idx - A_INST] + kb);
    };
    constexpr int INST = A_INST + B_INST;

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    // fp32 residual with whole-width wave tiles: the accumulators start from
    // the residual, read here ahead of the ring's first k-tiles, and the
    // epilogue only adds the bias and stores.  The residual read then
    // overlaps the main loop instead of joining the epilogue's write burst,
    // when every tile of a round finishes at once.  Registers hold rows of
    // the transposed blocks: row lrow + 32 i, columns 8 g + 4 h .. + 3 of
    // block j (the MFMA output layout); rows past M read zero.
    // The loads are unconditional (a wave that keeps the residual for its
    // epilogue gets an empty resource and reads zeros): a branch here would
    // make the compiler wait for the whole prologue before the first MFMA.
    // One workgroup per CU only: at two per CU (the 256 x 128 tiles) the
    // stack measured slower with it (MelBandRoformer 6.14 -> 6.22 ms per
    // chunk), against 15.53 -> 15.44 for the 256 x 256 BSRoformer stack.
    constexpr bool kResInAcc = EPI == kEpiRes && ACT == MSST_ACT_NONE &&
                               std::is_same<OutT, float>::value && MINB == 1;
    bool res_in_acc = false;
    if constexpr (kResInAcc) {
        res_in_acc = vec != 0 && n0 + wn * WN + WN <= N;
        const int wrow0 = __builtin_amdgcn_readfirstlane(m0 + wm * WM);
        const int nrows = res_in_acc ? max(0, min(M - wrow0, WM)) : 0;
        const float* rbase = uniform_ptr(reinterpret_cast<const float*>(residual) +
                                         (int64_t)max(wrow0, 0) * N);
        const int rbytes = __builtin_amdgcn_readfirstlane(nrows * N * 4);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = n0 + wn * WN + j * 32 + 8 * g + 4 * lhalf;
                    const f4 r = load16_bounded(rbase, rbytes, ((i * 32 + lrow) * N + c) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = r[e];
                }
    }

    // Activation epilogues (FF1): the accumulators start from the bias, so
    // the VALU-bound epilogue has one operation less per element (columns
    // past N, or no bias: zeros).
    constexpr bool kBiasInAcc = EPI == kEpiPlain && ACT != MSST_ACT_NONE;
    if constexpr (kBiasInAcc) {
        const float* bb = uniform_ptr(bias);
        const int bbytes = bias ? N * 4 : 0;
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = n0 + wn * WN + j * 32 + 8 * g + 4 * lhalf;
                const f4 b = load16_bounded(bb, bbytes, (uint32_t)c * 4u);
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = b[e];
            }
    }

    const int KT = K / BK;
    // Prologue: k-tiles 0 .. NSTG-1 fill the ring (clamped: short K
    // re-fetches the last tile, keeping the per-stage instruction count
    // fixed for vmcnt).
#pragma unroll
    for (int st = 0; st < NSTG; ++st)
#pragma unroll
        for (int idx = 0; idx < INST; ++idx) issue_one(idx, min(st, KT - 1) * BK, st);
    if constexpr (kResInAcc || kBiasInAcc) {
        // Take the residual / bias here, behind the ring's DMAs in the vmcnt queue:
        // the compiler's wait is then vmcnt(stages * instructions) instead of
        // vmcnt(0) at the main loop's entry.
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) use_now(acc[i][j]);
    }

    // Fragment reads of (k-tile, substep) pairs run one MFMA group ahead of
    // their use, across k-tile boundaries: the barrier that publishes k-tile
    // kt + 1 sits before the MFMAs of kt's last substep, so kt + 1's first
    // fragments are read while those MFMAs run.  After that barrier every
    // wave has finished reading slot kt % NSTG, which then receives the DMA
    // of k-tile kt + NSTG.
    h8 af[KK][MI], bf[KK][NI];
    auto load_frags = [&](int slot, int kk) {
        const half_t* As = lds[slot];
        const half_t* Bs = lds[slot] + BM * BK;
        const int c = kk * 2 + lhalf;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int r = wm * WM + i * 32 + lrow;
            af[kk][i] = *reinterpret_cast<const h8*>(As + r * BK + ((c ^ chunk_swz<BK>(r)) << 3));
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int r = wn * WN + j * 32 + lrow;
            bf[kk][j] = *reinterpret_cast<const h8*>(Bs + r * BK + ((c ^ chunk_swz<BK>(r)) << 3));
        }
    };
    // k-tile 0 has landed once at most the NSTG-1 newer k-tiles remain; in
    // the loop, k-tile kt + 1 once at most NSTG-2 remain (kt + NSTG is
    // issued after that wait).
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTG - 1) * INST) : "memory");
    lds_barrier();
    load_frags(0, 0);
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt % NSTG;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            if (kk + 1 < KK) {
                load_frags(cur, kk + 1);
            } else {
                // Unconditional (also on the last k-tile, where it reads a
                // stale slot that is never used), so the waits the compiler
                // places for this substep's fragments see one path only.
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTG - 2) * INST) : "memory");
                lds_barrier();
                // Past the end the DMA re-fetches the last k-tile into a slot
                // that is never read again (keeps every wait count equal).
                const int knext = min(kt + NSTG, KT - 1) * BK;
#pragma unroll
                for (int idx = 0; idx < INST; ++idx) issue_one(idx, knext, cur);
                load_frags((kt + 1) % NSTG, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = mfma32x32x16(bf[kk][j], af[kk][i], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();

    // acc holds the transposed blocks (W_j . A_i^T, see store_tile_lds).
    constexpr int kRegion = (int)(sizeof(lds) / sizeof(float) / NW);
    // Padded staging rows when a fragment row of them fits the wave's share
    // of the ring, else the unpadded swizzled layout.
    constexpr bool kSwz = 32 * (WN + 4) > kRegion;
    constexpr int kIP = pick_ip<MI, kSwz ? WN : WN + 4, kRegion>();
    static_assert(kIP * 32 * (kSwz ? WN : WN + 4) <= kRegion, "epilogue staging does not fit in LDS");
    if constexpr (kResInAcc) {
        if (res_in_acc) {
            store_tile_lds<MI, NI, kIP, kEpiPlain, OutT, true, ACT, kSwz>(
                acc, reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion, lane, m0 + wm * WM,
                n0 + wn * WN, M, N, bias, act, nullptr, out, vec != 0, rope);
            return;
        }
    }
    store_tile_lds<MI, NI, kIP, EPI, OutT, true, ACT, kSwz, kBiasInAcc>(acc, reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion,
                                           lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act,
                                           residual, out, vec != 0, rope);
}

// ---------------------------------------------------------------------------
// Ping-pong fp16 GEMM: 256 x 256 tiles, 8 waves in two groups of four (one
// wave of each group per SIMD), LDS-DMA ring of NSTG k-tiles of BK.
//
// Group g owns rows 128 g .. 128 g + 127 of the tile; within a group wave
// w % 4 owns 64 columns (a 128 x 64 wave tile of 4 x 2 32x32 blocks, as in
// gemm_f16_dma_kernel).  The groups run half a k-tile apart: while one
// group's waves issue the k-tile's MFMAs (at raised wave priority), the
// other group's waves read their next k-tile's fragments from LDS and issue
// their share of the ring's DMAs, so each SIMD's MFMA pipe is fed by one
// wave or the other at every moment.  Every phase ends at a workgroup
// barrier that both groups pass:
//
//   barrier:  B0    B1    B2    B3    B4   ...
//   group 0:  | mem 0 | mma 0 | mem 1 | mma 1 | ...
//   group 1:  |       | mem 0 | mma 0 | mem 1 | ...
//
// (group 1 passes one extra barrier before its loop).  The memory phase of
// k-tile t also issues the DMA of k-tile t + NSTG - 1 into the slot of
// t - 1, which both groups finished reading before barrier B(2t) (group 1
// reads t - 1 between B(2t - 1) and B(2t)).  Right after its memory phase
// of k-tile t (so before B(2t + 2), ahead of group 0's read of k-tile
// t + 1), every wave waits until its own DMAs of k-tile t + 1 have landed:
// each wave issues INST DMAs per k-tile, in k-tile order, and at that point
// the newest ones it has issued belong to k-tiles t + 2 .. t + NSTG - 1, so
// vmcnt((NSTG - 2) INST) leaves exactly those in flight.  Past the last
// k-tile the DMAs re-fetch it into the free slot (every wait count stays
// the same); the last wait of each wave is vmcnt(0), so no DMA is in flight
// when the epilogue stages through the ring (group 0 after B(2 KT), group 1
// after its last MFMAs; their staging regions are disjoint).
// ---------------------------------------------------------------------------
template <int BK, int NSTG, int EPI, int ACT, typename OutT>
__global__ __launch_bounds__(512, 1) void gemm_pp_kernel(
    const half_t* __restrict__ A, const half_t* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int M, int N, int K, int act, int tiles_n, int per_xcd,
    int vec, EpiRope rope) {
    constexpr int BM = 256, BN = 256, NW = 8;
    constexpr int CPR = BK / 8;              // 16-byte chunks per LDS row
    constexpr int RPD = 64 / CPR;            // rows per 1 KB DMA instruction
    constexpr int KK = BK / 16;              // MFMA k-substeps per k-tile
    constexpr int WM = 128, WN = 64;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_INST = BM / RPD / NW;    // DMA instructions per wave per k-tile
    constexpr int B_INST = BN / RPD / NW;
    constexpr int INST = A_INST + B_INST;
    constexpr int STAGE = (BM + BN) * BK;
    static_assert(A_INST * RPD * NW == BM && B_INST * RPD * NW == BN, "DMA split");
    static_assert(NSTG >= 2 && (NSTG - 1) * INST <= 63, "vmcnt range");
    __shared__ __attribute__((aligned(16))) half_t lds[NSTG][STAGE];

    int tm, tn;
    tile_coords(tiles_n, per_xcd, tm, tn, ((M + BM - 1) / BM) * tiles_n);
    if (tm < 0) return;
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave-uniform (readfirstlane: the group branch below is a scalar one).
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wid >> 2;
    const int wm = grp, wn = wid & 3;
    const int lrow = lane & 31, lhalf = lane >> 5;

    const int a_bytes = M * K * 2, b_bytes = N * K * 2;
    const int sub_row = lane / CPR;
    uint32_t aoff[A_INST], boff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int rl = (wid * A_INST + i) * RPD + sub_row;
        const int lchunk = (lane % CPR) ^ chunk_swz<BK>(rl);
        aoff[i] = (uint32_t)(min(m0 + rl, M - 1) * K + lchunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int rl = (wid * B_INST + i) * RPD + sub_row;
        const int lchunk = (lane % CPR) ^ chunk_swz<BK>(rl);
        boff[i] = (uint32_t)(min(n0 + rl, N - 1) * K + lchunk * 8) * 2u;
    }
    auto issue = [&](int k0, int slot) {  // this wave's INST DMAs of the k-tile at k0
        const uint32_t kb = (uint32_t)k0 * 2u;
#pragma unroll
        for (int i = 0; i < A_INST; ++i)
            dma16(A, a_bytes, lds[slot] + (wid * A_INST + i) * 512, aoff[i] + kb);
#pragma unroll
        for (int i = 0; i < B_INST; ++i)
            dma16(W, b_bytes, lds[slot] + BM * BK + (wid * B_INST + i) * 512, boff[i] + kb);
    };

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    // Accumulators that start from the fp32 residual (whole-width wave
    // tiles) or from the bias (activation epilogues), read ahead of the
    // ring's first DMAs as in gemm_f16_dma_kernel.
    constexpr bool kResInAcc = EPI == kEpiRes && ACT == MSST_ACT_NONE &&
                               std::is_same<OutT, float>::value;
    constexpr bool kBiasInAcc = EPI == kEpiPlain && ACT != MSST_ACT_NONE;
    bool res_in_acc = false;
    if constexpr (kResInAcc) {
        res_in_acc = vec != 0 && n0 + wn * WN + WN <= N;
        const int wrow0 = __builtin_amdgcn_readfirstlane(m0 + wm * WM);
        const int nrows = res_in_acc ? max(0, min(M - wrow0, WM)) : 0;
        const float* rbase = uniform_ptr(reinterpret_cast<const float*>(residual) +
                                         (int64_t)max(wrow0, 0) * N);
        const int rbytes = __builtin_amdgcn_readfirstlane(nrows * N * 4);
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int c = n0 + wn * WN + j * 32 + 8 * g + 4 * lhalf;
                    const f4 r = load16_bounded(rbase, rbytes, ((i * 32 + lrow) * N + c) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = r[e];
                }
    }
    if constexpr (kBiasInAcc) {
        const float* bb = uniform_ptr(bias);
        const int bbytes = bias ? N * 4 : 0;
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int c = n0 + wn * WN + j * 32 + 8 * g + 4 * lhalf;
                const f4 b = load16_bounded(bb, bbytes, (uint32_t)c * 4u);
#pragma unroll
                for (int i = 0; i < MI; ++i)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][4 * g + e] = b[e];
            }
    }

    const int KT = K / BK;
    // Prologue: k-tiles 0 .. NSTG-2 (clamped for short K: the last k-tile
    // is re-fetched, which keeps the per-k-tile DMA count fixed).
#pragma unroll
    for (int st = 0; st < NSTG - 1; ++st) issue(min(st, KT - 1) * BK, st);
    if constexpr (kResInAcc || kBiasInAcc) {
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int j = 0; j < NI; ++j) use_now(acc[i][j]);
    }

    h8 af[KK][MI], bf[KK][NI];
    auto mem_phase = [&](int t) {
        const int slot = t % NSTG;
        const half_t* As = lds[slot];
        const half_t* Bs = lds[slot] + BM * BK;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const int c = kk * 2 + lhalf;
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int r = wm * WM + i * 32 + lrow;
                af[kk][i] = *reinterpret_cast<const h8*>(As + r * BK + ((c ^ chunk_swz<BK>(r)) << 3));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const int r = wn * WN + j * 32 + lrow;
                bf[kk][j] = *reinterpret_cast<const h8*>(Bs + r * BK + ((c ^ chunk_swz<BK>(r)) << 3));
            }
        }
        const int tn2 = t + NSTG - 1;
        issue(min(tn2, KT - 1) * BK, tn2 % NSTG);
    };
    auto mma_phase = [&]() {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = mfma32x32x16(bf[kk][j], af[kk][i], acc[i][j]);
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Own DMAs of the next k-tile landed (the last wait drains the ring).
    auto wait_next = [&](int t) {
        if (t + 1 < KT)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTG - 2) * INST) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    };

    // Both groups run the same loop body (one copy of the code: separate
    // loops per group made the register allocator shuffle and spill the
    // accumulators); group 1 passes one barrier before it, group 0 one
    // after it, so group 1 runs one phase behind.
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NSTG - 2) * INST) : "memory");  // k-tile 0
    if (grp == 1) lds_barrier();  // B(0)
    for (int t = 0; t < KT; ++t) {
        lds_barrier();  // group 0: B(2t), group 1: B(2t + 1)
        mem_phase(t);
        wait_next(t);
        lds_barrier();  // group 0: B(2t + 1), group 1: B(2t + 2)
        mma_phase();
    }
    if (grp == 0) lds_barrier();  // B(2 KT)

    constexpr int kRegion = (int)(sizeof(lds) / sizeof(float) / NW);
    constexpr bool kSwz = 32 * (WN + 4) > kRegion;
    constexpr int kIP = pick_ip<MI, kSwz ? WN : WN + 4, kRegion>();
    static_assert(kIP * 32 * (kSwz ? WN : WN + 4) <= kRegion, "epilogue staging does not fit in LDS");
    float* region = reinterpret_cast<float*>(&lds[0][0]) + wid * kRegion;
    if constexpr (kResInAcc) {
        if (res_in_acc) {
            store_tile_lds<MI, NI, kIP, kEpiPlain, OutT, true, ACT, kSwz>(
                acc, region, lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act, nullptr, out,
                vec != 0, rope);
            return;
        }
    }
    store_tile_lds<MI, NI, kIP, EPI, OutT, true, ACT, kSwz, kBiasInAcc>(
        acc, region, lane, m0 + wm * WM, n0 + wn * WN, M, N, bias, act, residual, out, vec != 0,
        rope);
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
// Skinny GEMM, vector form (N <= NP, K <= 64 * VA * S, 16-byte aligned rows):
// HBM-bound.  One wave per row, two rows in flight; lane l covers the
// 16-byte A slices l, l + 64, .. (VA elements each, S slices).  The lane's
// slices of the N weight rows are loaded once and stay in
// registers for every row the wave visits, so per row only the row itself
// is read.  fp16 A and W use v_dot2_f32_f16 on packed pairs.  The N partial
// dots go through gate_sums8 (8 at a time): sum n ends in lanes 8n .. 8n + 7
// and lane 8n applies the bias (loaded once) and the activation and writes
// output n.  The grid is sized so each wave sees many rows (the weight
// loads are paid once per wave).
// ---------------------------------------------------------------------------
template <typename AT, typename WT, typename OutT, int NP, int S>
__global__ __launch_bounds__(kThreads) void gemm_skinny_vec_kernel(
    const AT* __restrict__ A, const WT* __restrict__ W, const float* __restrict__ bias,
    const OutT* residual, OutT* out, int64_t M, int N, int K, int act) {
    constexpr int VA = 16 / (int)sizeof(AT);
    constexpr bool kDot2 = sizeof(AT) == 2 && sizeof(WT) == 2;
    constexpr int WW = VA * (int)sizeof(WT) / 4;  // 32-bit words per weight slice: 2, 4 or 8
    static_assert(NP == 8 || NP == 16, "NP");
    const int lane = threadIdx.x & 63;
    // Wave-uniform row index: keeps the buffer descriptors in SGPRs (a
    // per-lane descriptor would need a waterfall loop around every load).
    const int64_t wave = (int64_t)blockIdx.x * (kThreads / 64) +
                         __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * (kThreads / 64);
    // Weight slices: w[s][n] holds W[n, (s * 64 + lane) * VA ..][VA] as raw
    // words, zero past N or K (buffer loads past the row read zero).
    uint32_t w[S][NP][WW];
#pragma unroll
    for (int n = 0; n < NP; ++n) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<WT*>(W) + (n < N ? (int64_t)n * K : 0), (short)0,
            n < N ? K * (int)sizeof(WT) : 0, 0x00020000);
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int off = ((s * 64 + lane) * VA) * (int)sizeof(WT);
            if constexpr (WW == 2) {
                const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
                w[s][n][0] = v[0];
                w[s][n][1] = v[1];
            } else {
#pragma unroll
                for (int q = 0; q < WW / 4; ++q) {
                    const u4v v = __builtin_bit_cast(
                        u4v, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * q, 0, 0));
#pragma unroll
                    for (int j = 0; j < 4; ++j) w[s][n][4 * q + j] = v[j];
                }
            }
        }
    }
    const int g = lane >> 3;
    float bl[NP / 8];
#pragma unroll
    for (int h = 0; h < NP / 8; ++h) bl[h] = (bias && 8 * h + g < N) ? bias[8 * h + g] : 0.0f;

    auto load_row = [&](int64_t row, u4v (&a)[S]) {
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<AT*>(A) + (row < M ? row : 0) * K, (short)0,
            row < M ? K * (int)sizeof(AT) : 0, 0x00020000);
#pragma unroll
        for (int s = 0; s < S; ++s)
            a[s] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(
                                               r, ((s * 64 + lane) * VA) * (int)sizeof(AT), 0, 0));
    };
    auto wval = [&](int s, int n, int e) -> float {  // element e of weight slice (s, n)
        if constexpr (sizeof(WT) == 2)
            return (float)__builtin_bit_cast(h2, w[s][n][e / 2])[e % 2];
        else
            return __builtin_bit_cast(float, w[s][n][e]);
    };
    auto finish = [&](int64_t row, const u4v (&a)[S]) {
        float acc[NP];
#pragma unroll
        for (int n = 0; n < NP; ++n) {
            float d = 0.0f;
#pragma unroll
            for (int s = 0; s < S; ++s) {
                if constexpr (kDot2) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // Copy the vector element out first: clang's
                        // __builtin_bit_cast of an ext_vector element lvalue
                        // reads element 0 whatever the index.
                        const uint32_t ae = a[s][e];
                        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, ae),
                                                   __builtin_bit_cast(h2, w[s][n][e]), d, false);
                    }
                } else if constexpr (sizeof(AT) == 2) {
                    const h8 x = __builtin_bit_cast(h8, a[s]);
#pragma unroll
                    for (int e = 0; e < VA; ++e) d = fmaf((float)x[e], wval(s, n, e), d);
                } else {
                    const f4 x = __builtin_bit_cast(f4, a[s]);
#pragma unroll
                    for (int e = 0; e < VA; ++e) d = fmaf(x[e], wval(s, n, e), d);
                }
            }
            acc[n] = d;
        }
#pragma unroll
        for (int h = 0; h < NP / 8; ++h) {
            float part[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) part[i] = acc[8 * h + i];
            const float tot = gate_sums8(part, lane);
            const int n = 8 * h + g;
            if ((lane & 7) == 0 && n < N && row < M) {
                float v = act_apply(tot + bl[h], act);
                const int64_t idx = row * (int64_t)N + n;
                if (residual) v += (float)residual[idx];
                out[idx] = (OutT)v;
            }
        }
    };
    u4v a0[S], a1[S];
    for (int64_t row = wave; row < M; row += 2 * nwaves) {
        load_row(row, a0);
        load_row(row + nwaves, a1);
        finish(row, a0);
        finish(row + nwaves, a1);
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

template <typename OutT>
int vec_flag(const OutT* res, const OutT* out, int N) {
    return (N % 4 == 0 && aligned(out, 4 * sizeof(OutT)) && aligned(res, 4 * sizeof(OutT))) ? 1
                                                                                            : 0;
}

template <int BM, int BN, typename OutT>
int launch_f16(const void* x, bool x_f32, const half_t* w, const float* bias,
               const OutT* res, OutT* out, int M, int N, int K, int act, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int per_xcd;
    int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    const int vec = vec_flag(res, out, N);
#define MSST_L16(AF, RS)                                                                        \
    hipLaunchKernelGGL((gemm_f16_kernel<BM, BN, AF, RS, OutT>), dim3(grid), dim3(kThreads), 0, s, \
                       x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd, vec)
    if (x_f32) {
        if (res) MSST_L16(true, true); else MSST_L16(true, false);
    } else {
        if (res) MSST_L16(false, true); else MSST_L16(false, false);
    }
#undef MSST_L16
    return check_launch("gemm_f16_kernel");
}

template <int BM, int BN, int BK, int NSTG, int MINB, int NWN, int EPI, int ACT, typename OutT>
void launch_dma_epi(const half_t* x, const half_t* w, const float* bias, const OutT* res,
                    OutT* out, int M, int N, int K, int act, hipStream_t s, const EpiRope& rope) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int per_xcd;
    const int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    hipLaunchKernelGGL((gemm_f16_dma_kernel<BM, BN, BK, NSTG, MINB, NWN, EPI, ACT, OutT>),
                       dim3(grid), dim3(128 * NWN), 0, s, x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd,
                       vec_flag(res, out, N), rope);
}

template <int BK, int NSTG, int EPI, int ACT, typename OutT>
void launch_pp_epi(const half_t* x, const half_t* w, const float* bias, const OutT* res,
                   OutT* out, int M, int N, int K, int act, hipStream_t s, const EpiRope& rope) {
    const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    int per_xcd;
    const int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    hipLaunchKernelGGL((gemm_pp_kernel<BK, NSTG, EPI, ACT, OutT>), dim3(grid), dim3(512), 0, s, x,
                       w, bias, res, out, M, N, K, act, tiles_n, per_xcd, vec_flag(res, out, N),
                       rope);
}

template <int BK, int NSTG, typename OutT>
int launch_pp(const half_t* x, const half_t* w, const float* bias, const OutT* res, OutT* out,
              int M, int N, int K, int act, hipStream_t s, const EpiRope* rope = nullptr) {
    if (rope) {
        if constexpr (std::is_same<OutT, half_t>::value)
            launch_pp_epi<BK, NSTG, kEpiRope, MSST_ACT_NONE, OutT>(x, w, bias, res, out, M, N, K,
                                                                   act, s, *rope);
        else
            return set_error(MSST_ERR_UNSUPPORTED, "RoPE epilogue needs fp16 output");
    } else if (act == MSST_ACT_GELU && !res) {
        launch_pp_epi<BK, NSTG, kEpiPlain, MSST_ACT_GELU, OutT>(x, w, bias, res, out, M, N, K, act,
                                                                s, EpiRope{});
    } else if (act != MSST_ACT_NONE) {
        return set_error(MSST_ERR_UNSUPPORTED, "ping-pong GEMM takes no activation but GELU");
    } else if (res) {
        launch_pp_epi<BK, NSTG, kEpiRes, MSST_ACT_NONE, OutT>(x, w, bias, res, out, M, N, K, act,
                                                              s, EpiRope{});
    } else {
        launch_pp_epi<BK, NSTG, kEpiPlain, MSST_ACT_NONE, OutT>(x, w, bias, res, out, M, N, K, act,
                                                                s, EpiRope{});
    }
    return check_launch("gemm_pp_kernel");
}

// The activation is a template parameter of the kernel (its epilogue is
// straight-line code per activation).
template <int BM, int BN, int BK, int NSTG, int MINB, int NWN, int EPI, typename OutT>
void launch_dma_act(const half_t* x, const half_t* w, const float* bias, const OutT* res,
                    OutT* out, int M, int N, int K, int act, hipStream_t s, const EpiRope& rope) {
    switch (act) {
        case MSST_ACT_GELU:
            launch_dma_epi<BM, BN, BK, NSTG, MINB, NWN, EPI, MSST_ACT_GELU, OutT>(x, w, bias, res, out,
                                                                             M, N, K, act, s, rope);
            break;
        case MSST_ACT_SIGMOID:
            launch_dma_epi<BM, BN, BK, NSTG, MINB, NWN, EPI, MSST_ACT_SIGMOID, OutT>(
                x, w, bias, res, out, M, N, K, act, s, rope);
            break;
        case MSST_ACT_SILU:
            launch_dma_epi<BM, BN, BK, NSTG, MINB, NWN, EPI, MSST_ACT_SILU, OutT>(x, w, bias, res, out,
                                                                             M, N, K, act, s, rope);
            break;
        default:
            launch_dma_epi<BM, BN, BK, NSTG, MINB, NWN, EPI, MSST_ACT_NONE, OutT>(x, w, bias, res, out,
                                                                             M, N, K, act, s, rope);
    }
}

template <int BM, int BN, int BK, int NSTG, int MINB, int NWN, typename OutT>
int launch_f16_dma(const half_t* x, const half_t* w, const float* bias, const OutT* res,
                   OutT* out, int M, int N, int K, int act, hipStream_t s,
                   const EpiRope* rope = nullptr) {
    if (rope) {
        if constexpr (std::is_same<OutT, half_t>::value) {
            if (act != MSST_ACT_NONE)
                return set_error(MSST_ERR_UNSUPPORTED, "RoPE epilogue takes no activation");
            launch_dma_epi<BM, BN, BK, NSTG, MINB, NWN, kEpiRope, MSST_ACT_NONE, OutT>(
                x, w, bias, res, out, M, N, K, act, s, *rope);
        } else {
            return set_error(MSST_ERR_UNSUPPORTED, "RoPE epilogue needs fp16 output");
        }
    } else if (res) {
        launch_dma_act<BM, BN, BK, NSTG, MINB, NWN, kEpiRes, OutT>(x, w, bias, res, out, M, N, K, act,
                                                              s, EpiRope{});
    } else {
        launch_dma_act<BM, BN, BK, NSTG, MINB, NWN, kEpiPlain, OutT>(x, w, bias, res, out, M, N, K, act,
                                                                s, EpiRope{});
    }
    return check_launch("gemm_f16_dma_kernel");
}

template <int BM, int BN, typename OutT>
int launch_f32(const void* x, bool x_f16, const float* w, const float* bias,
               const OutT* res, OutT* out, int M, int N, int K, int act, hipStream_t s) {
    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int per_xcd;
    int grid = num_xcd_slots((int64_t)tiles_m * tiles_n, per_xcd);
    const int vec = vec_flag(res, out, N);
    if (!x_f16 && K % 32 == 0 && aligned(x, 16) && aligned(w, 16) &&
        (int64_t)M * K * 4 < ((int64_t)1 << 31) && (int64_t)N * K * 4 < ((int64_t)1 << 31)) {
        const float* xf = reinterpret_cast<const float*>(x);
        if (res)
            hipLaunchKernelGGL((gemm_f32_dma_kernel<BM, BN, 16, true, OutT>), dim3(grid), dim3(kThreads),
                               0, s, xf, w, bias, res, out, M, N, K, act, tiles_n, per_xcd, vec);
        else
            hipLaunchKernelGGL((gemm_f32_dma_kernel<BM, BN, 16, false, OutT>), dim3(grid), dim3(kThreads),
                               0, s, xf, w, bias, res, out, M, N, K, act, tiles_n, per_xcd, vec);
        return check_launch("gemm_f32_dma_kernel");
    }
#define MSST_L32(AH, RS)                                                                        \
    hipLaunchKernelGGL((gemm_f32_kernel<BM, BN, AH, RS, OutT>), dim3(grid), dim3(kThreads), 0, s, \
                       x, w, bias, res, out, M, N, K, act, tiles_n, per_xcd, vec)
    if (x_f16) {
        if (res) MSST_L32(true, true); else MSST_L32(true, false);
    } else {
        if (res) MSST_L32(false, true); else MSST_L32(false, false);
    }
#undef MSST_L32
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
        constexpr int VA = 16 / (int)sizeof(AT);
        const int slices = (K + 64 * VA - 1) / (64 * VA);
        if (K % VA == 0 && aligned(x, 16) && aligned(w, 16) && slices <= 2) {
            // Vector form: whole 16-byte A slices per lane, weights in
            // registers; about 16 rows per wave (1024 blocks of 4 waves for
            // M = 49662).
            const int64_t vblocks = std::max<int64_t>(1, std::min<int64_t>((M + 63) / 64, 1024));
#define MSST_SKV(NP, S)                                                                       \
    hipLaunchKernelGGL((gemm_skinny_vec_kernel<AT, WT, OutT, NP, S>), dim3((unsigned)vblocks), \
                       dim3(kThreads), 0, s, a, wt, bias, res, out, M, N, K, act)
            if (N <= 8) {
                if (slices == 1) MSST_SKV(8, 1); else MSST_SKV(8, 2);
            } else {
                if (slices == 1) MSST_SKV(16, 1); else MSST_SKV(16, 2);
            }
#undef MSST_SKV
            return check_launch("gemm_skinny_vec_kernel");
        }
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
        // LDS-DMA fast path: f16 operands, whole 64-wide k-tiles, 32-bit
        // buffer offsets.
        const bool dma_ok = !x_f32 && K % 64 == 0 && aligned(x, 16) && aligned(w, 16) &&
                            (M + 256) * K * 2 < ((int64_t)1 << 31) &&
                            (N + 256) * K * 2 < ((int64_t)1 << 31);
        if (dma_ok) {
            const half_t* xh = reinterpret_cast<const half_t*>(x);
            const half_t* wh = reinterpret_cast<const half_t*>(w);
            // Tile choice (measured on the Roformer shapes): with sigmoid or
            // SiLU the epilogue is VALU-heavy and 128 x 128 tiles at three
            // workgroups per CU hide it behind the others' main loops;
            // otherwise one 256 x 256 tile per CU (8 waves) moves the fewest
            // L2 -> LDS bytes per flop, run by the ping-pong kernel (6-8 %
            // faster than gemm_f16_dma_kernel on the same tiles, with
            // bit-identical results; fp16 residuals keep the latter, whose
            // epilogue residual fits the register budget).  N = 128 (mod 256)
            // takes 256 x 128 tiles at two workgroups per CU instead of padding
            // a quarter of the 256-wide tiles (MelBandRoformer out-proj / FF2
            // 9-10 % faster), unless N = 384 takes the 192 x 384 tiles below.
            // (The activation kernels start their accumulators from 16-byte
            // bias loads, which need N % 4 == 0; other N take the
            // register-staged kernel below.)
            // 128 x 128 tiles at three workgroups per CU also take:
            //  - launches with fewer 256 x 256 tiles than CUs (small M):
            //    M = 1000, K = N = 512 with residual 22 -> 8.5 us;
            //  - the K <= 512 residual GEMM (the out-projection): its
            //    epilogue residual then streams beside other workgroups'
            //    main loops (58.5 against 61 us alone; BSRoformer chunk
            //    15.28 -> 15.23 ms, MelBandRoformer 6.19 -> 6.16 ms, A/B
            //    in the stack on one box).
            const bool small = ((M + 255) / 256) * ((N + 255) / 256) < 256;
            const bool narrow_res = res != nullptr && K <= 512;
            // N = 384 (MelBandRoformer's dim): whole-width 192 x 384 tiles, 12
            // waves of 96 x 64, three per SIMD.  The bytes fetched per flop of
            // a 256 x 256 tile (where 256 x 128 fetches 1.5 times as many), and
            // M = 48060 makes 251 tiles: one round on 256 CUs.  At one tile per
            // CU a short last round runs alone (K = 1536 with residual: 259
            // tiles 118 us against 77 us for 256 tiles; 93 us on 256 x 128
            // tiles), so they are taken when the last round is empty or holds
            // at least 64 tiles.  The rule ignores K, although with K = 384 the
            // 128 x 128 x 3 tiles are faster past one round (M = 192240: 160
            // against 186 us): a batch of MelBandRoformer chunks (M = 4 x
            // 48060) then takes the tiles of one chunk and computes the same
            // bits (these tiles start their accumulators from the residual,
            // the others add it in the epilogue).
            const int64_t t384 = ((int64_t)M + 191) / 192;
            const bool fit384 = t384 % 256 == 0 || t384 % 256 >= 64;
            if (act == MSST_ACT_NONE && N == 384 && !small && fit384)
                return launch_f16_dma<192, 384, 32, 3, 1, 6, OutT>(xh, wh, bias, res, o, m, n, k, act,
                                                                   s);
            if (act == MSST_ACT_NONE && (small || narrow_res) && N % 4 == 0)
                return launch_f16_dma<128, 128, 32, 3, 3, 2, OutT>(xh, wh, bias, res, o, m, n, k, act,
                                                                   s);
            if (act == MSST_ACT_NONE && N % 256 == 0 && (!res || std::is_same<OutT, float>::value))
                return launch_pp<32, 3, OutT>(xh, wh, bias, res, o, m, n, k, act, s);
            // GELU without residual (the feed-forward's first linear) on the
            // ping-pong tiles too: with the 11-operation GELU and non-temporal
            // output stores, FF1 170 -> 158 us alone and the BSRoformer chunk
            // 15.06 -> 14.96 ms in the stack (interleaved A/Bs on two boxes).
            if (act == MSST_ACT_GELU && !res && !small && N % 256 == 0)
                return launch_pp<32, 3, OutT>(xh, wh, bias, res, o, m, n, k, act, s);
            if (act != MSST_ACT_NONE && N % 4 == 0)
                return launch_f16_dma<128, 128, 32, 3, 3, 2, OutT>(xh, wh, bias, res, o, m, n, k, act,
                                                                   s);
            if (act == MSST_ACT_NONE && N % 256 == 128)
                return launch_f16_dma<256, 128, 32, 3, 2, 2, OutT>(xh, wh, bias, res, o, m, n, k, act,
                                                                   s);
            if (act == MSST_ACT_NONE)
                return launch_f16_dma<256, 256, 32, 3, 1, 4, OutT>(xh, wh, bias, res, o, m, n, k, act,
                                                                   s);
        }
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

extern "C" int msst_linear_rope(const void* x, const void* w, const float* bias, void* out,
                                int64_t M, int64_t K, int64_t N, const float* cos_t,
                                const float* sin_t, int64_t rope_cols, int64_t dim_head,
                                int64_t pos_div, int64_t pos_mod, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && w && out && cos_t && sin_t, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(M >= 0 && K > 0 && N > 0, MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(dim_head > 0 && dim_head % 4 == 0 && rope_cols >= 0 && rope_cols <= N &&
                     rope_cols % 64 == 0 && rope_cols % dim_head == 0,
                 MSST_ERR_INVALID_ARG,
                 "rope_cols must be a multiple of 64 and of dim_head (a multiple of 4), <= N");
    MSST_REQUIRE(pos_div >= 1 && pos_mod >= 1 && pos_div < (1 << 24) && pos_mod < (1 << 24),
                 MSST_ERR_INVALID_ARG, "bad position divisor / modulus");
    MSST_REQUIRE(K % 64 == 0 && M < (1 << 24) && (M + 256) * K * 2 < ((int64_t)1 << 31) &&
                     (N + 256) * K * 2 < ((int64_t)1 << 31),
                 MSST_ERR_UNSUPPORTED, "shape outside the fused RoPE GEMM (K % 64, M < 2^24)");
    MSST_REQUIRE(aligned(x, 16) && aligned(w, 16) && aligned(out, 16) && aligned(bias, 4) &&
                     aligned(cos_t, 8) && aligned(sin_t, 8),
                 MSST_ERR_ALIGNMENT, "x, w, out must be 16-byte and cos/sin 8-byte aligned");
    if (M == 0) return MSST_OK;
    EpiRope r{};
    r.cos = cos_t;
    r.sin = sin_t;
    r.cols = (int)rope_cols;
    r.dh = (int)dim_head;
    r.div = (int)pos_div;
    r.mod = (int)pos_mod;
    r.inv_div = 1.0f / (float)pos_div;
    r.inv_mod = 1.0f / (float)pos_mod;
    const half_t* xh = reinterpret_cast<const half_t*>(x);
    const half_t* wh = reinterpret_cast<const half_t*>(w);
    half_t* oh = reinterpret_cast<half_t*>(out);
    // Fewer 256 x 256 tiles than CUs (small M): 128 x 128 tiles at three
    // workgroups per CU (the 64-column wave tiles divide the RoPE columns).
    if (((M + 255) / 256) * ((N + 255) / 256) < 256)
        return launch_f16_dma<128, 128, 32, 3, 3, 2, half_t>(xh, wh, bias, nullptr, oh, (int)M,
                                                             (int)N, (int)K, MSST_ACT_NONE,
                                                             as_stream(stream), &r);
    if (N % 256 == 0)
        return launch_pp<32, 3, half_t>(xh, wh, bias, nullptr, oh, (int)M, (int)N, (int)K,
                                        MSST_ACT_NONE, as_stream(stream), &r);
    return launch_f16_dma<256, 256, 32, 3, 1, 4, half_t>(xh, wh, bias, nullptr, oh, (int)M,
                                                         (int)N, (int)K, MSST_ACT_NONE,
                                                         as_stream(stream), &r);
}
