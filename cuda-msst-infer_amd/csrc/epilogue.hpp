// epilogue.hpp — epilogue of the MFMA GEMM kernels (gemm.hip): LDS-staged,
// row-contiguous stores with bias, activation, residual or RoPE applied on
// the way out.
#pragma once

#include "msst_common.hpp"

namespace msst {
namespace {

template <typename T>
__device__ __forceinline__ f4 ld4(const T* p);
template <>
__device__ __forceinline__ f4 ld4<float>(const float* p) { return *reinterpret_cast<const f4*>(p); }
template <>
__device__ __forceinline__ f4 ld4<half_t>(const half_t* p) {
    h4 v = *reinterpret_cast<const h4*>(p);
    return f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
template <typename T>
__device__ __forceinline__ void st4(T* p, f4 v);
template <>
__device__ __forceinline__ void st4<float>(float* p, f4 v) { *reinterpret_cast<f4*>(p) = v; }
template <>
__device__ __forceinline__ void st4<half_t>(half_t* p, f4 v) {
    *reinterpret_cast<h4*>(p) = h4{(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
}

// Largest divisor IP of MI whose IP*32 x WN fp32 block fits a wave's
// REGION floats of LDS.
template <int MI, int WN, int REGION>
constexpr int pick_ip() {
    int ip = MI;
    while (ip > 1 && (ip * 32 * WN > REGION || MI % ip != 0)) --ip;
    return ip;
}

// Epilogue variants of store_tile_lds.
constexpr int kEpiPlain = 0;  // act(acc + bias)
constexpr int kEpiRes = 1;    // act(acc + bias) + residual
constexpr int kEpiRope = 2;   // rotary embedding on the first `cols` columns

// Interleaved-pair RoPE applied by the epilogue (ops_misc.cu:39-69 on the
// q/k head columns): the output is rounded to fp16 first, as the reference
// rotates the fp16 tensor the linear wrote, and rotated in fp32.  The
// position of row r is (r / div) % mod; cos/sin are [positions, dh / 2].
struct EpiRope {
    const float* cos;
    const float* sin;
    int cols;  // columns [0, cols) are rotated (a multiple of dh)
    int dh;    // head dim (pairs per position: dh / 2)
    int div, mod;
    float inv_div, inv_mod;
};

// Epilogue through LDS.  A wave's (MI*32) x (NI*32) accumulator block is
// written to its LDS region IP fragment-rows at a time (static register
// indices).  TR = false: acc[i][j] = A_i . W_j^T (register v of lane l holds
// row 8 (v / 4) + 4 h + v % 4, column l % 32), one 4-byte write per value.
// TR = true: acc[i][j] = W_j . A_i^T, the transposed block (register v holds
// row l % 32, column 8 (v / 4) + 4 h + v % 4), so every 4 registers are 4
// consecutive columns of one row: one 16-byte write each, into rows padded
// by 4 floats so the 16 rows a b128 pass writes fall in distinct banks.
// Each wave stages through its own region, and a wave's LDS operations
// execute in order, so no barrier is needed inside the epilogue.
//
// The block is read back row-contiguously: each lane owns 4 consecutive
// columns, so bias is loaded once and global stores are 16-byte (f32) /
// 8-byte (f16) and row-contiguous.  The read-back runs in batches of U rows
// per lane, fully unrolled.  The global loads of batch b + 1 (residual
// rows, or RoPE cos/sin rows) are issued before the stores of batch b: loads
// and stores share one in-order vmcnt on CDNA, so a load issued after a
// batch of stores could only be waited for together with those stores.
// Whole-width wave tiles (the common case) store through buffer resources
// bounded to the rows below M, so the read-back loop has no per-row branch:
// with branches, the compiler's conservative wait at each join made every
// store wait for all earlier ones (a full memory round trip per store).
// EPI and ACT are compile-time (ACT < 0: the runtime `act` argument).
// Caller: the wave's region is free (after a barrier that follows the last
// read of the k-loop's tiles).
// SWZ (with TR): unpadded LDS rows of WN floats, the 16-byte chunk c of row
// r stored at chunk c ^ (r % (WN / 4)), for callers whose region has no room
// for the padding; reads stay conflict-free, writes see at most two-way
// conflicts.
// NOBIAS: the accumulators already hold the bias (no add here).
// UMAX: rows per lane and batch at most (fewer keep fewer residual rows in
// flight, for kernels that need the registers).
template <int MI, int NI, int IP, int EPI, typename OutT, bool TR = false, int ACT = -1,
          bool SWZ = false, bool NOBIAS = false, int UMAX = 8>
__device__ __forceinline__ void store_tile_lds(f16x (&acc)[MI][NI], float* wlds, int lane,
                                               int row0, int col0, int M, int N,
                                               const float* __restrict__ bias, int act,
                                               const OutT* residual, OutT* out, bool vec,
                                               const EpiRope& rope = EpiRope{}) {
    static_assert(MI % IP == 0, "IP must divide MI");
    static_assert(!SWZ || TR, "the swizzled layout is for the transposed blocks");
    constexpr int WN = NI * 32;
    constexpr int LDW = TR ? (SWZ ? WN : WN + 4) : WN;  // LDS row stride (floats)
    constexpr int CMASK = WN / 4 - 1;
    // Float offset of the 16-byte chunk holding column c (a multiple of 4) of row r.
    auto at = [&](int r, int c) { return r * LDW + (SWZ ? (((c >> 2) ^ (r & CMASK)) << 2) : c); };
    constexpr int LPR = WN / 4;    // lanes per row
    constexpr int RPI = 64 / LPR;  // rows per iteration
    constexpr int ITERS = IP * 32 / RPI;
    constexpr int U = ITERS >= UMAX ? UMAX : ITERS;
    static_assert(ITERS % U == 0, "batch must divide the row count");
    constexpr int BPP = ITERS / U;        // batches per pass
    constexpr int NB = (MI / IP) * BPP;   // batches in total
    constexpr bool LOADS = EPI == kEpiRes || EPI == kEpiRope;
    const int lrow = lane & 31, lh = lane >> 5;
    const int rr = lane / LPR, cq = lane % LPR;
    const int col = col0 + cq * 4;
    // Wave-uniform: the whole wave tile lies inside N with aligned rows, so
    // only one of the store paths below ever executes for a wave.
    const bool full = vec && col0 + WN <= N;
    // Wave-uniform as well: rope.cols is a multiple of the 64-column wave
    // tile whenever the host selects this epilogue.
    const bool rope_on = EPI == kEpiRope && col0 + WN <= rope.cols;
    const int pair = EPI == kEpiRope ? (col % rope.dh) >> 1 : 0;
    f4 bv = f4{0.0f, 0.0f, 0.0f, 0.0f};
    if (bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e) bv[e] = (col + e < N) ? bias[col + e] : 0.0f;
    }
    auto local_row = [&](int b, int u) {  // row of batch b, slot u within the wave tile
        return (b / BPP) * IP * 32 + ((b % BPP) * U + u) * RPI + rr;
    };
    auto batch_row = [&](int b, int u) { return row0 + local_row(b, u); };
    // Stage pass p (fragment rows p*IP .. p*IP+IP-1) into the region.
    auto stage = [&](int p) {
#pragma unroll
        for (int ii = 0; ii < IP; ++ii)
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                if constexpr (TR) {
#pragma unroll
                    for (int g = 0; g < 4; ++g) {
                        const f16x& a = acc[p * IP + ii][j];
                        *reinterpret_cast<f4*>(wlds + at(ii * 32 + lrow, j * 32 + 8 * g + 4 * lh)) =
                            f4{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
                    }
                } else {
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        const int r = ii * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                        wlds[r * LDW + j * 32 + lrow] = acc[p * IP + ii][j][v];
                    }
                }
            }
    };
    auto finish = [&](f4 v, const f4& rv) {  // bias, activation, residual / RoPE
        f4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if constexpr (ACT >= 0)
                o[e] = act_fixed<ACT>(NOBIAS ? v[e] : v[e] + bv[e]);
            else
                o[e] = act_apply(v[e] + bv[e], act);
        }
        if constexpr (EPI == kEpiRes) o += rv;
        if constexpr (EPI == kEpiRope) {
            if (rope_on) {
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float a = (float)(half_t)o[2 * e];
                    const float bb = (float)(half_t)o[2 * e + 1];
                    o[2 * e] = a * rv[e] - bb * rv[2 + e];
                    o[2 * e + 1] = a * rv[2 + e] + bb * rv[e];
                }
            }
        }
        return o;
    };
    auto rope_batch = [&](int b, f4 (&rv)[U]) {  // (cos, cos, sin, sin) of the lane's 2 pairs
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int grow = min(batch_row(b, u), M - 1);
            int rem, pos;
            const int q = divmod24(grow, rope.div, rope.inv_div, rem);
            divmod24(q, rope.mod, rope.inv_mod, pos);
            const int t = pos * (rope.dh >> 1) + pair;
            const float2 c = *reinterpret_cast<const float2*>(rope.cos + t);
            const float2 sn = *reinterpret_cast<const float2*>(rope.sin + t);
            rv[u] = f4{c.x, c.y, sn.x, sn.y};
        }
    };

    if (full) {
        // Whole-width wave tile: buffer accesses bounded to the wave's rows
        // below M, so rows past M read zero and their stores are dropped by
        // the hardware.  The loop is then straight-line code, and each wait
        // the compiler places covers exactly the data it needs: no per-row
        // branch forces a wait for every earlier store.
        // row0 is wave-uniform; readfirstlane keeps the resources in SGPRs.
        const int wrow0 = __builtin_amdgcn_readfirstlane(row0);
        const int nrows = max(0, min(M - wrow0, MI * 32));
        const int64_t rbase = (int64_t)max(wrow0, 0) * N;
        const int nbytes = __builtin_amdgcn_readfirstlane(nrows * N * (int)sizeof(OutT));
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr(out + rbase), (short)0, nbytes, 0x00020000);
        __amdgpu_buffer_rsrc_t rr_src = ro;
        if constexpr (EPI == kEpiRes)
            rr_src = __builtin_amdgcn_make_buffer_rsrc(
                uniform_ptr(const_cast<OutT*>(residual) + rbase), (short)0, nbytes, 0x00020000);
        auto off = [&](int b, int u) { return (local_row(b, u) * N + col) * (int)sizeof(OutT); };
        auto load_res = [&](int b, f4 (&rv)[U]) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if constexpr (std::is_same<OutT, float>::value) {
                    rv[u] = __builtin_bit_cast(
                        f4, __builtin_amdgcn_raw_buffer_load_b128(rr_src, off(b, u), 0, 0));
                } else {
                    const h4 h = __builtin_bit_cast(
                        h4, __builtin_amdgcn_raw_buffer_load_b64(rr_src, off(b, u), 0, 0));
                    rv[u] = f4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
                }
            }
        };
        f4 rb[2][U];
        if constexpr (EPI == kEpiRes) load_res(0, rb[0]);
        if constexpr (EPI == kEpiRope) {
            if (rope_on) rope_batch(0, rb[0]);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b % BPP == 0) stage(b / BPP);
            if (b + 1 < NB) {
                if constexpr (EPI == kEpiRes) load_res(b + 1, rb[(b + 1) & 1]);
                if constexpr (EPI == kEpiRope) {
                    if (rope_on) rope_batch(b + 1, rb[(b + 1) & 1]);
                }
            }
            // Activation epilogues (the feed-forward's first linear: 203 MB of
            // fp16 output per BSRoformer layer) store non-temporally, so the
            // output stream does not evict the A and W lines the other tiles
            // still read from L2 (FF1 178 -> 168 us alone, BSRoformer chunk
            // 15.11 -> 14.93 ms in an interleaved A/B; same results).
            constexpr int kStorePolicy = ACT > 0 ? 2 : 0;  // nt
            const int it0 = (b % BPP) * U;
            f4 v[U];
#pragma unroll
            for (int u = 0; u < U; ++u)
                v[u] = *reinterpret_cast<const f4*>(wlds + at((it0 + u) * RPI + rr, cq * 4));
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const f4 o = finish(v[u], rb[b & 1][u]);
                if constexpr (std::is_same<OutT, float>::value) {
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, o), ro, off(b, u),
                                                           0, kStorePolicy);
                } else {
                    const h4 h = h4{(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
                    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, h), ro, off(b, u),
                                                          0, kStorePolicy);
                }
            }
        }
        return;
    }
    // rv: residual values, or (cos, cos, sin, sin) of the lane's 2 pairs.
    auto load_batch = [&](int b, f4 (&rv)[U]) {
        if constexpr (EPI == kEpiRes) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int grow = batch_row(b, u);
                const int64_t idx = (int64_t)grow * N + col;
                rv[u] = f4{0.0f, 0.0f, 0.0f, 0.0f};
                if (grow < M) {
                    if (full) {
                        rv[u] = ld4<OutT>(residual + idx);
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (col + e < N) rv[u][e] = (float)residual[idx + e];
                    }
                }
            }
        } else if constexpr (EPI == kEpiRope) {
            if (rope_on) rope_batch(b, rv);
        }
    };
    f4 rbuf[2][U];
    if constexpr (LOADS) load_batch(0, rbuf[0]);
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int p = b / BPP;
        if (b % BPP == 0) stage(p);
        if constexpr (LOADS) {
            if (b + 1 < NB) load_batch(b + 1, rbuf[(b + 1) & 1]);
        }
        const int it0 = (b % BPP) * U;
        f4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            v[u] = *reinterpret_cast<const f4*>(wlds + at((it0 + u) * RPI + rr, cq * 4));
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int grow = batch_row(b, u);
            if (grow < M) {
                const f4 o = finish(v[u], rbuf[b & 1][u]);
                const int64_t idx = (int64_t)grow * N + col;
                if (full) {
                    st4<OutT>(out + idx, o);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (col + e < N) out[idx + e] = (OutT)o[e];
                }
            }
        }
    }
}

}  // namespace
}  // namespace msst
