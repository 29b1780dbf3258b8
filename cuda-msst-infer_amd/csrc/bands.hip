// bands.hip — the band split and the mask estimator of the Roformer models
// as grouped kernels.
//
// The reference runs both as a host loop over the bands (BSRoformer
// model_bs_roformer.cu:337-368 and :374-414; MelBandRoformer
// model_mel_band_roformer.cu:658-690 and :696-738): per band an rms_norm and
// a linear (band split), or a linear -> tanh -> ... -> linear chain and a
// glu (mask estimator), then stack / cat.  With 60-62 bands of 801 tokens
// each, every one of those GEMMs is a handful of tiles, so here each layer
// is ONE launch over all bands:
//
//   band_norm_kernel     segmented RMSNorm: band b of every token row,
//                        scaled by sqrt(dims[b]), written as fp16 and
//                        zero-padded to a multiple of 64 columns (the fp16
//                        rounding is the cast ops::linear applies to its
//                        input, ops_linear.cu:155).
//   band_gemm_kernel     grouped MFMA GEMM (LDS DMA ring, 128 x 128 tiles),
//                        one group per band; the tile -> band map is a scan
//                        over the bands' tile counts.  Epilogues:
//                          kSplit   out[r, b, :] = acc + bias_b       (fp32)
//                          kHidden  tanh(acc + bias)                  (fp16,
//                                   tanh_fast: msst_common.hpp)
//                          kGlu     v[m] * sigmoid(v[m + d])          (fp32)
//                        For kGlu the W rows are read interleaved (tile row
//                        2m is W row m, 2m + 1 is W row m + d), so each GLU
//                        pair lands in adjacent columns of one lane.
//
// Per-band weights stay in the caller's tensors: msst_band_plan_init copies
// their addresses and the band offsets into a device-resident plan once per
// model (and packs the band-split weights, whose widths are not multiples of
// the 64-column k-slice, into zero-padded rows).  The per-chunk calls read
// the plan with scalar loads.
#include <algorithm>
#include <cstring>
#include <vector>

#include "msst_common.hpp"

namespace msst {
namespace {

constexpr int kMaxBands = 64;
constexpr int kMaxLinears = 8;

struct BandPlan {
    int nb, dim, hid, L;
    int ftot;        // sum of dims
    int kpad_total;  // sum of kpad
    int has_split, has_mask;
    int fd[kMaxBands];    // features of band b (2 * freqs * channels)
    int foff[kMaxBands];  // first feature column of band b
    int kpad[kMaxBands];  // fd rounded up to 64
    int koff[kMaxBands];  // first column of band b in the padded layout
    const float* split_gamma[kMaxBands];
    const half_t* split_w[kMaxBands];  // caller's W_b [dim, fd_b], read once by the packer
    const float* split_b[kMaxBands];
    const half_t* mask_w[kMaxBands * kMaxLinears];
    const float* mask_b[kMaxBands * kMaxLinears];
    // STFT side: n_idx = ftot / 2 band feature pairs over nbins = F * ch
    // interleaved bins; `identity` when pair j is bin j (no averaging).
    int ch, F, nbins, n_idx, identity;
    int64_t idx_off;  // byte offset of the index tables in the plan
};
// Plan layout: header | packed band-split weights (band b is [dim][kpad_b]
// halves at element offset dim * koff_b) | fidx [n_idx] | csr_off [nbins + 1]
// | csr_list [n_idx] (int32; csr lists, per bin g, the pairs j with
// fidx[j] == g in ascending order).
constexpr int64_t kPlanHeader = (sizeof(BandPlan) + 255) / 256 * 256;

__device__ __forceinline__ const half_t* packed_w(const BandPlan* p) {
    return reinterpret_cast<const half_t*>(reinterpret_cast<const char*>(p) + kPlanHeader);
}
__device__ __forceinline__ const int* plan_ints(const BandPlan* p) {
    return reinterpret_cast<const int*>(reinterpret_cast<const char*>(p) + p->idx_off);
}

// ---------------------------------------------------------------------------
// W_b [dim, fd_b] -> packed [dim, kpad_b], zero beyond fd_b.  One thread per
// packed element; grid-stride over all bands.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void band_pack_kernel(BandPlan* plan, int nb, int dim,
                                                        int64_t total) {
    half_t* dst = reinterpret_cast<half_t*>(reinterpret_cast<char*>(plan) + kPlanHeader);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        // Find the band of packed element i (bands are few; linear scan).
        int b = 0;
        while (b + 1 < nb && i >= (int64_t)dim * plan->koff[b + 1]) ++b;
        const int64_t local = i - (int64_t)dim * plan->koff[b];
        const int kp = plan->kpad[b], fd = plan->fd[b];
        const int n = (int)(local / kp), k = (int)(local % kp);
        dst[i] = k < fd ? plan->split_w[b][(int64_t)n * fd + k] : (half_t)0.0f;
    }
}

// ---------------------------------------------------------------------------
// Segmented RMSNorm: one wave per (token row, band).
//   y[r, koff_b + j] = fp16(x[r, foff_b + j] * rsqrt(sum_j x^2 + 1e-12)
//                            * gamma_b[j] * sqrt(fd_b)),   0 for fd_b <= j < kpad_b
// (ops_norm.cu:85-111 with scale = sqrt(band dim), model_bs_roformer.cu:357).
// ---------------------------------------------------------------------------
constexpr int kNormMaxPerLane = 16;  // fd <= 1024

__global__ __launch_bounds__(256) void band_norm_kernel(const BandPlan* __restrict__ plan,
                                                        const float* __restrict__ x, int rows,
                                                        half_t* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int64_t gw = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = plan->nb;
    const int row = (int)(gw / nb), b = (int)(gw % nb);
    if (row >= rows) return;
    const int fd = plan->fd[b], kp = plan->kpad[b];
    const float* xr = x + (int64_t)row * plan->ftot + plan->foff[b];
    const float* g = plan->split_gamma[b];
    float v[kNormMaxPerLane];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kNormMaxPerLane; ++i) {
        const int j = lane + 64 * i;
        v[i] = j < fd ? xr[j] : 0.0f;
        ss = fmaf(v[i], v[i], ss);
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss + 1e-12f);
    const float scale = sqrtf((float)fd);
    half_t* yr = y + (int64_t)row * plan->kpad_total + plan->koff[b];
#pragma unroll
    for (int i = 0; i < kNormMaxPerLane; ++i) {
        const int j = lane + 64 * i;
        if (j < kp) yr[j] = j < fd ? (half_t)(v[i] * inv * g[j] * scale) : (half_t)0.0f;
    }
}

// ---------------------------------------------------------------------------
// Grouped GEMM over bands.
// ---------------------------------------------------------------------------
constexpr int kSplit = 0, kHidden = 1, kGlu = 2;
constexpr int kBM = 128, kBN = 128, kBK = 32, kStages = 3;
constexpr int kGemmThreads = 256;

struct BandGemmArgs {
    const BandPlan* plan;
    const half_t* a;  // A buffer
    int a_bytes;
    int lda;          // elements between A rows
    int a_band;       // elements between bands' A blocks (kSplit: unused, koff)
    int K;            // kHidden / kGlu: K of every band
    int layer;        // MLP layer index (weights mask_w[b * L + layer])
    int M;            // token rows
    void* out;
    int ldo;
    int o_band;       // kHidden: elements between bands' output blocks
    int tiles_m;
    int per_xcd;      // tiles per XCD (the grid is 8 * per_xcd workgroups)
};

// Tile t -> (band, tm, tn) and the band's N.
template <int MODE>
__device__ __forceinline__ int find_band(const BandGemmArgs& a, int t, int& b, int& tm, int& tn) {
    const BandPlan* p = a.plan;
    const int nb = p->nb;
    int n;
    if constexpr (MODE == kGlu) {
        int start = 0;
        b = -1;
        for (int g = 0; g < nb; ++g) {
            const int ng = 2 * p->fd[g];
            const int cnt = a.tiles_m * ((ng + kBN - 1) / kBN);
            if (t < start + cnt) {
                b = g;
                n = ng;
                t -= start;
                break;
            }
            start += cnt;
        }
        if (b < 0) return 0;
    } else {
        n = MODE == kSplit ? p->dim : p->hid;
        const int per = a.tiles_m * ((n + kBN - 1) / kBN);
        b = t / per;
        if (b >= nb) return 0;
        t -= b * per;
    }
    const int tiles_n = (n + kBN - 1) / kBN;
    tm = t / tiles_n;
    tn = t % tiles_n;
    return n;
}

template <int MODE>
__global__ __launch_bounds__(kGemmThreads, 3) void band_gemm_kernel(BandGemmArgs args) {
    constexpr int CPR = kBK / 8;           // 16-byte chunks per LDS row (4)
    constexpr int RPD = 64 / CPR;          // rows per 1 KB DMA instruction (16)
    constexpr int KK = kBK / 16;           // MFMA k-substeps per k-tile
    constexpr int WM = kBM / 2, WN = kBN / 2;
    constexpr int MI = WM / 32, NI = WN / 32;
    constexpr int A_INST = kBM / RPD / 4, B_INST = kBN / RPD / 4;  // per wave
    constexpr int INST = A_INST + B_INST;
    constexpr int STAGE = (kBM + kBN) * kBK;
    __shared__ __attribute__((aligned(16))) half_t lds[kStages][STAGE];

    // XCD-aware: workgroups are dealt round-robin to the 8 XCDs, so
    // workgroup w takes tile (w % 8) * per_xcd + w / 8 and each XCD walks a
    // contiguous run of tiles -- a few bands at a time, whose W stays in
    // that XCD's L2.
    const int t = (int)(blockIdx.x & 7) * args.per_xcd + (int)(blockIdx.x >> 3);
    int b, tm, tn;
    const int N = find_band<MODE>(args, t, b, tm, tn);
    if (N == 0) return;
    const BandPlan* plan = args.plan;
    const int M = args.M;
    const int m0 = tm * kBM, n0 = tn * kBN;

    // Band operands.
    int K, a_off;
    const half_t* W;
    const float* bias;
    int glu_d = 0;
    if constexpr (MODE == kSplit) {
        K = plan->kpad[b];
        a_off = plan->koff[b];
        W = packed_w(plan) + (int64_t)plan->dim * plan->koff[b];
        bias = plan->split_b[b];
    } else {
        K = args.K;
        a_off = b * args.a_band;
        W = plan->mask_w[b * plan->L + args.layer];
        bias = plan->mask_b[b * plan->L + args.layer];
        if constexpr (MODE == kGlu) glu_d = plan->fd[b];
    }

    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int wm = wid >> 1, wn = wid & 1;
    const int lrow = lane & 31, lhalf = lane >> 5;
    const int sub_row = lane / CPR;
    const int w_bytes = N * K * 2;

    uint32_t aoff[A_INST], boff[B_INST];
#pragma unroll
    for (int i = 0; i < A_INST; ++i) {
        const int rl = (wid * A_INST + i) * RPD + sub_row;
        const int lchunk = (lane % CPR) ^ ((rl >> 2) & 3);
        const int r = min(m0 + rl, M - 1);
        aoff[i] = (uint32_t)((int64_t)a_off + (int64_t)r * args.lda + lchunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < B_INST; ++i) {
        const int rl = (wid * B_INST + i) * RPD + sub_row;
        const int lchunk = (lane % CPR) ^ ((rl >> 2) & 3);
        int r = min(n0 + rl, N - 1);
        if constexpr (MODE == kGlu) r = (r >> 1) + (r & 1) * glu_d;  // interleave GLU pairs
        boff[i] = (uint32_t)(r * K + lchunk * 8) * 2u;
    }
    auto issue = [&](int k0, int buf) {
        const uint32_t kb = (uint32_t)k0 * 2u;
#pragma unroll
        for (int i = 0; i < A_INST; ++i)
            dma16(args.a, args.a_bytes, lds[buf] + (wid * A_INST + i) * 512, aoff[i] + kb);
#pragma unroll
        for (int i = 0; i < B_INST; ++i)
            dma16(W, w_bytes, lds[buf] + kBM * kBK + (wid * B_INST + i) * 512, boff[i] + kb);
    };

    f16x acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j) acc[i][j] = f16x{};

    const int KT = K / kBK;
#pragma unroll
    for (int st = 0; st < kStages - 1; ++st) issue(min(st, KT - 1) * kBK, st);
    for (int kt = 0; kt < KT; ++kt) {
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((kStages - 2) * INST) : "memory");
        lds_barrier();
        // Refill the slot read at kt - 1 (past the end: re-fetch the last
        // k-tile into a slot nothing reads again, keeping counts uniform).
        issue(min(kt + kStages - 1, KT - 1) * kBK, (kt + kStages - 1) % kStages);
        const half_t* As = lds[kt % kStages];
        const half_t* Bs = As + kBM * kBK;
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
            const int c = kk * 2 + lhalf;
            h8 af[MI], bf[NI];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int r = wm * WM + i * 32 + lrow;
                af[i] = *reinterpret_cast<const h8*>(As + r * kBK + ((c ^ ((r >> 2) & 3)) << 3));
            }
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const int r = wn * WN + j * 32 + lrow;
                bf[j] = *reinterpret_cast<const h8*>(Bs + r * kBK + ((c ^ ((r >> 2) & 3)) << 3));
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j) acc[i][j] = mfma32x32x16(bf[j], af[i], acc[i][j]);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_barrier();

    // Epilogue: acc[i][j] = W_j . A_i^T, so register 4 g + e of lane l is row
    // l % 32, column 8 g + 4 (l / 32) + e of block (i, j).  Each 32-row
    // fragment row goes through the wave's LDS region (rows padded by 4
    // floats) and is read back as 4 consecutive columns per lane.  Stores go
    // through a buffer resource based at the wave's first row, with the
    // offset of an invalid row or column replaced by one past the resource
    // (the hardware drops the store): no per-row branch, so the compiler's
    // waits are exact instead of one full memory round trip per store.
    constexpr int LDW = WN + 4;
    constexpr int LPR = WN / 4;      // lanes per row (16)
    constexpr int RPI = 64 / LPR;    // rows per read (4)
    constexpr int ROWS = 32 / RPI;   // reads per fragment row (8)
    float* wl = reinterpret_cast<float*>(&lds[0][0]) + wid * (32 * LDW);
    static_assert(4 * 32 * LDW * 4 <= (int)sizeof(lds), "epilogue staging does not fit");
    const int rr = lane / LPR, cq = lane % LPR;
    const int col = n0 + wn * WN + cq * 4;  // first of the lane's 4 columns
    f4 bv;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        int c = min(col + e, N - 1);
        if constexpr (MODE == kGlu) c = (c >> 1) + (c & 1) * glu_d;
        bv[e] = bias[c];
    }
    const int wrow = __builtin_amdgcn_readfirstlane(m0 + wm * WM);
    const int nrows = max(0, min(M - wrow, WM));
    // Base (element) of the wave's first row in the band's output columns.
    int64_t base;
    int esize;
    if constexpr (MODE == kSplit) {
        base = (int64_t)wrow * args.ldo + b * plan->dim;
        esize = 4;
    } else if constexpr (MODE == kHidden) {
        base = (int64_t)b * args.o_band + (int64_t)wrow * args.ldo;
        esize = 2;
    } else {
        base = (int64_t)wrow * args.ldo + plan->foff[b];
        esize = 4;
    }
    char* const obase = uniform_ptr(reinterpret_cast<char*>(args.out) + base * esize);
    // The resource spans the wave's rows below M (whole output rows).
    const int span = __builtin_amdgcn_readfirstlane(nrows * args.ldo * esize);
    const __amdgpu_buffer_rsrc_t ro =
        __builtin_amdgcn_make_buffer_rsrc(obase, (short)0, span, 0x00020000);
    const uint32_t kDrop = 0x80000000u;  // past any resource here (span < 2^31)
    const bool col_ok = col < N;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g)
                *reinterpret_cast<f4*>(wl + lrow * LDW + j * 32 + 8 * g + 4 * lhalf) =
                    f4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                       acc[i][j][4 * g + 3]};
        f4 v[ROWS];
#pragma unroll
        for (int it = 0; it < ROWS; ++it)
            v[it] = *reinterpret_cast<const f4*>(wl + (it * RPI + rr) * LDW + cq * 4) + bv;
#pragma unroll
        for (int it = 0; it < ROWS; ++it) {
            const int lr = i * 32 + it * RPI + rr;  // row within the wave tile
            const bool ok = col_ok && lr < nrows;
            if constexpr (MODE == kSplit) {
                // N = dim is a multiple of 4: the 4 columns are valid together.
                const uint32_t off = ok ? (uint32_t)((lr * args.ldo + col) * 4) : kDrop;
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4v, v[it]), ro, off, 0, 0);
            } else if constexpr (MODE == kHidden) {
                const uint32_t off = ok ? (uint32_t)((lr * args.ldo + col) * 2) : kDrop;
                const h4 h = h4{(half_t)tanh_fast(v[it][0]), (half_t)tanh_fast(v[it][1]),
                                (half_t)tanh_fast(v[it][2]), (half_t)tanh_fast(v[it][3])};
                __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2v, h), ro, off, 0, 0);
            } else {
                // Columns (col, col + 1) and (col + 2, col + 3) are GLU pairs
                // m = col / 2, col / 2 + 1 (N = 2 d is even and col is a
                // multiple of 4, so a lane's pairs are whole).
                const float g0 = v[it][0] * (1.0f / (1.0f + expf(-v[it][1])));
                const float g1 = v[it][2] * (1.0f / (1.0f + expf(-v[it][3])));
                const uint32_t off = ok ? (uint32_t)((lr * args.ldo + (col >> 1)) * 4) : kDrop;
                const uint32_t off1 = (ok && col + 2 < N) ? off + 4u : kDrop;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(g0), ro, off, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(g1), ro, off1, 0, 0);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// STFT <-> band features.  Both kernels move [.., frames, pairs] <-> [.., bins,
// frames] through a 64 x 64 LDS tile (float2 = one complex value), so global
// reads and writes are both contiguous along their fastest axis.
// ---------------------------------------------------------------------------
constexpr int kTile = 64;

// out[b, t, j] = stft[b * ch + s, f, t] with f * ch + s = fidx[j].
// Grid (frame tiles, pair tiles, batch).
__global__ __launch_bounds__(256) void band_gather_kernel(const BandPlan* __restrict__ plan,
                                                          const float2* __restrict__ stft,
                                                          int T, float2* __restrict__ out) {
    __shared__ float2 tile[kTile][kTile + 1];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * kTile, j0 = blockIdx.y * kTile, b = blockIdx.z;
    const int ch = plan->ch, F = plan->F, n = plan->n_idx;
    const int* fidx = plan_ints(plan);
#pragma unroll 4
    for (int it = 0; it < kTile / 4; ++it) {
        const int jj = it * 4 + (tid >> 6), tt = tid & 63;
        const int j = j0 + jj, t = t0 + tt;
        float2 v = float2{0.0f, 0.0f};
        if (j < n && t < T) {
            const int g = fidx[j];
            const int f = g / ch, sc = g - f * ch;
            v = stft[((int64_t)(b * ch + sc) * F + f) * T + t];
        }
        tile[jj][tt] = v;
    }
    __syncthreads();
#pragma unroll 4
    for (int it = 0; it < kTile / 4; ++it) {
        const int tt = it * 4 + (tid >> 6), jj = tid & 63;
        const int j = j0 + jj, t = t0 + tt;
        if (j < n && t < T) out[((int64_t)b * T + t) * n + j] = tile[jj][tt];
    }
}

// Per mask row (stem, batch, frame): the mean over the pairs that hold each
// bin, mg[row, g] = sum_{j in csr(g)} masks[row, j] / max(count, 1e-8)
// (scatter_add then the clamped division).  Grid (bin blocks, rows).
__global__ __launch_bounds__(256) void mask_mean_kernel(const BandPlan* __restrict__ plan,
                                                        const float2* __restrict__ masks,
                                                        float2* __restrict__ mg) {
    const int nbins = plan->nbins, n = plan->n_idx;
    const int g = blockIdx.x * 256 + threadIdx.x;
    if (g >= nbins) return;
    const int* ints = plan_ints(plan);
    const int* off = ints + n;
    const int* list = off + nbins + 1;
    const int64_t row = blockIdx.y;
    const float2* mr = masks + row * n;
    float2 acc = float2{0.0f, 0.0f};
    const int k0 = off[g], k1 = off[g + 1];
    for (int k = k0; k < k1; ++k) {
        const float2 v = mr[list[k]];
        acc.x += v.x;
        acc.y += v.y;
    }
    const float den = fmaxf((float)(k1 - k0), 1e-8f);
    mg[row * nbins + g] = float2{acc.x / den, acc.y / den};
}

// out[(b * stems + n) * ch + s, f, t] = stft[b * ch + s, f, t] * m[n, b, t, g]
// (complex), g = f * ch + s; bin 0 zeroed when zero_dc.  m is [stems][batch,
// frames, nbins].  Grid (frame tiles, bin tiles, stems * batch).
__global__ __launch_bounds__(256) void mask_apply_kernel(const BandPlan* __restrict__ plan,
                                                         const float2* __restrict__ m,
                                                         const float2* __restrict__ stft,
                                                         int batch, int T, int zero_dc,
                                                         float2* __restrict__ out) {
    __shared__ float2 tile[kTile][kTile + 1];
    const int tid = threadIdx.x;
    const int t0 = blockIdx.x * kTile, g0 = blockIdx.y * kTile;
    const int nb = blockIdx.z;  // stem-major: n * batch + b
    const int n = nb / batch, b = nb - n * batch;
    const int ch = plan->ch, F = plan->F, nbins = plan->nbins;
    const int stems = gridDim.z / batch;
    const float2* mrow = m + (int64_t)nb * T * nbins;
#pragma unroll 4
    for (int it = 0; it < kTile / 4; ++it) {
        const int tt = it * 4 + (tid >> 6), gg = tid & 63;
        const int t = t0 + tt, g = g0 + gg;
        tile[gg][tt] = (t < T && g < nbins) ? mrow[(int64_t)t * nbins + g] : float2{0.0f, 0.0f};
    }
    __syncthreads();
#pragma unroll 4
    for (int it = 0; it < kTile / 4; ++it) {
        const int gg = it * 4 + (tid >> 6), tt = tid & 63;
        const int t = t0 + tt, g = g0 + gg;
        if (t < T && g < nbins) {
            const int f = g / ch, sc = g - f * ch;
            const float2 x = stft[((int64_t)(b * ch + sc) * F + f) * T + t];
            const float2 k = tile[gg][tt];
            float2 o = float2{x.x * k.x - x.y * k.y, x.x * k.y + x.y * k.x};
            if (zero_dc && f == 0) o = float2{0.0f, 0.0f};
            out[((int64_t)((b * stems + n) * ch + sc) * F + f) * T + t] = o;
        }
    }
}

int gemm_tiles_split(const BandPlan& h, int tiles_m) {
    return h.nb * tiles_m * ((h.dim + kBN - 1) / kBN);
}

}  // namespace
}  // namespace msst

using namespace msst;

namespace {

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return MSST_OK;
    return set_error(MSST_ERR_LAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}

// Host mirror of the plan header, validated against the config.
int fill_plan(const msst_band_config* c, BandPlan& h) {
    MSST_REQUIRE(c, MSST_ERR_INVALID_ARG, "null config");
    MSST_REQUIRE(c->num_bands >= 1 && c->num_bands <= kMaxBands && c->band_dims,
                 MSST_ERR_UNSUPPORTED, "1..64 bands");
    MSST_REQUIRE(c->dim >= 64 && c->dim % 64 == 0, MSST_ERR_UNSUPPORTED,
                 "dim must be a multiple of 64");
    MSST_REQUIRE(c->mlp_linears >= 1 && c->mlp_linears <= kMaxLinears, MSST_ERR_UNSUPPORTED,
                 "1..8 mask-estimator linears");
    MSST_REQUIRE(c->mlp_linears == 1 || (c->hidden >= 64 && c->hidden % 64 == 0),
                 MSST_ERR_UNSUPPORTED, "hidden width must be a multiple of 64");
    memset(&h, 0, sizeof(h));
    h.nb = c->num_bands;
    h.dim = c->dim;
    h.hid = c->mlp_linears > 1 ? c->hidden : 0;
    h.L = c->mlp_linears;
    int f = 0, k = 0;
    for (int b = 0; b < h.nb; ++b) {
        const int d = c->band_dims[b];
        MSST_REQUIRE(d >= 2 && d <= 1024 && d % 2 == 0, MSST_ERR_UNSUPPORTED,
                     "band dims must be even and in [2, 1024]");
        h.fd[b] = d;
        h.foff[b] = f;
        h.kpad[b] = (d + 63) / 64 * 64;
        h.koff[b] = k;
        f += d;
        k += h.kpad[b];
    }
    h.ftot = f;
    h.kpad_total = k;
    h.n_idx = f / 2;
    h.ch = c->audio_channels;
    h.F = c->stft_bins;
    h.identity = c->freq_indices == nullptr;
    if (h.ch > 0 || h.F > 0) {
        MSST_REQUIRE((h.ch == 1 || h.ch == 2) && h.F >= 1, MSST_ERR_UNSUPPORTED,
                     "STFT side needs 1 or 2 channels and stft_bins >= 1");
        h.nbins = h.F * h.ch;
        if (h.identity)
            MSST_REQUIRE(h.n_idx == h.nbins, MSST_ERR_INVALID_ARG,
                         "without freq_indices the bands must cover every bin once");
        else
            for (int j = 0; j < h.n_idx; ++j)
                MSST_REQUIRE(c->freq_indices[j] >= 0 && c->freq_indices[j] < h.nbins,
                             MSST_ERR_INVALID_ARG, "freq_indices out of range");
    }
    h.idx_off = kPlanHeader + ((int64_t)h.dim * h.kpad_total * 2 + 255) / 256 * 256;
    return MSST_OK;
}

int64_t plan_bytes(const BandPlan& h) {
    return h.idx_off + 4 * ((int64_t)h.n_idx * 2 + h.nbins + 1);
}

}  // namespace

extern "C" int64_t msst_band_plan_bytes(const msst_band_config* c) {
    BandPlan h;
    if (fill_plan(c, h) != MSST_OK) return -1;
    return plan_bytes(h);
}

extern "C" int msst_band_plan_init(const msst_band_config* c, const float* const* split_gamma,
                                   const void* const* split_w, const float* const* split_b,
                                   const void* const* mask_w, const float* const* mask_b,
                                   void* plan, int64_t plan_bytes, void* stream) {
    BandPlan h;
    int rc = fill_plan(c, h);
    if (rc != MSST_OK) return rc;
    MSST_REQUIRE(plan && aligned(plan, 256), MSST_ERR_ALIGNMENT, "plan must be 256-byte aligned");
    MSST_REQUIRE(plan_bytes >= msst_band_plan_bytes(c), MSST_ERR_WORKSPACE, "plan too small");
    h.has_split = split_w != nullptr;
    h.has_mask = mask_w != nullptr;
    MSST_REQUIRE(!h.has_split || (split_gamma && split_b), MSST_ERR_INVALID_ARG,
                 "band split needs gamma, W and bias per band");
    MSST_REQUIRE(!h.has_mask || mask_b, MSST_ERR_INVALID_ARG, "mask estimator needs biases");
    for (int b = 0; b < h.nb; ++b) {
        if (h.has_split) {
            MSST_REQUIRE(split_gamma[b] && split_w[b] && split_b[b], MSST_ERR_INVALID_ARG,
                         "null band-split tensor");
            h.split_gamma[b] = split_gamma[b];
            h.split_w[b] = reinterpret_cast<const half_t*>(split_w[b]);
            h.split_b[b] = split_b[b];
        }
        if (h.has_mask)
            for (int l = 0; l < h.L; ++l) {
                const int i = b * h.L + l;
                MSST_REQUIRE(mask_w[i] && mask_b[i] && aligned(mask_w[i], 16),
                             MSST_ERR_ALIGNMENT, "mask weights must be non-null, 16-byte aligned");
                h.mask_w[i] = reinterpret_cast<const half_t*>(mask_w[i]);
                h.mask_b[i] = mask_b[i];
            }
    }
    hipStream_t s = as_stream(stream);
    // The header is copied from host memory before the call returns
    // (synchronous with respect to the host), then the packing kernel runs.
    rc = hip_status(hipMemcpy(plan, &h, sizeof(h), hipMemcpyHostToDevice), "plan upload");
    if (rc != MSST_OK) return rc;
    if (h.nbins > 0) {
        // fidx, then the inverse map as CSR (bins in order, pairs ascending).
        std::vector<int> ints((size_t)h.n_idx * 2 + h.nbins + 1, 0);
        int* fidx = ints.data();
        int* off = fidx + h.n_idx;
        int* list = off + h.nbins + 1;
        for (int j = 0; j < h.n_idx; ++j) fidx[j] = h.identity ? j : c->freq_indices[j];
        for (int j = 0; j < h.n_idx; ++j) ++off[fidx[j] + 1];
        for (int g = 0; g < h.nbins; ++g) off[g + 1] += off[g];
        std::vector<int> fill(off, off + h.nbins);
        for (int j = 0; j < h.n_idx; ++j) list[fill[fidx[j]]++] = j;
        rc = hip_status(hipMemcpy(reinterpret_cast<char*>(plan) + h.idx_off, ints.data(),
                                  ints.size() * sizeof(int), hipMemcpyHostToDevice),
                        "plan index upload");
        if (rc != MSST_OK) return rc;
    }
    if (h.has_split) {
        const int64_t total = (int64_t)h.dim * h.kpad_total;
        hipLaunchKernelGGL(band_pack_kernel, dim3(1024), dim3(256), 0, s,
                           reinterpret_cast<BandPlan*>(plan), h.nb, h.dim, total);
        rc = check_launch("band_pack_kernel");
        if (rc != MSST_OK) return rc;
        return hip_status(hipStreamSynchronize(s), "band_pack_kernel");
    }
    return MSST_OK;
}

extern "C" int64_t msst_band_split_workspace(const msst_band_config* c, int64_t rows) {
    BandPlan h;
    if (fill_plan(c, h) != MSST_OK || rows < 0) return -1;
    return (rows * h.kpad_total * 2 + 255) / 256 * 256;
}

extern "C" int msst_band_split(const msst_band_config* c, const void* plan, const float* x,
                               int64_t rows, float* out, void* workspace, int64_t ws_bytes,
                               void* stream) {
    BandPlan h;
    int rc = fill_plan(c, h);
    if (rc != MSST_OK) return rc;
    MSST_REQUIRE(plan && x && out && workspace, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(rows >= 0 && rows < (1 << 24), MSST_ERR_UNSUPPORTED, "rows out of range");
    MSST_REQUIRE(ws_bytes >= msst_band_split_workspace(c, rows), MSST_ERR_WORKSPACE,
                 "workspace too small");
    MSST_REQUIRE(rows * h.kpad_total * 2 < ((int64_t)1 << 31), MSST_ERR_UNSUPPORTED,
                 "normalised input exceeds 2^31 bytes");
    MSST_REQUIRE(aligned(out, 16) && aligned(workspace, 16), MSST_ERR_ALIGNMENT,
                 "out / workspace must be 16-byte aligned");
    if (rows == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const BandPlan* p = reinterpret_cast<const BandPlan*>(plan);
    half_t* y = reinterpret_cast<half_t*>(workspace);
    const int64_t waves = rows * h.nb;
    hipLaunchKernelGGL(band_norm_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p, x,
                       (int)rows, y);
    rc = check_launch("band_norm_kernel");
    if (rc != MSST_OK) return rc;
    BandGemmArgs a{};
    a.plan = p;
    a.a = y;
    a.a_bytes = (int)(rows * h.kpad_total * 2);
    a.lda = h.kpad_total;
    a.M = (int)rows;
    a.out = out;
    a.ldo = h.nb * h.dim;
    a.tiles_m = (int)((rows + kBM - 1) / kBM);
    const int tiles = gemm_tiles_split(h, a.tiles_m);
    a.per_xcd = (tiles + 7) / 8;
    hipLaunchKernelGGL(band_gemm_kernel<kSplit>, dim3((unsigned)(8 * a.per_xcd)),
                       dim3(kGemmThreads), 0, s, a);
    return check_launch("band_gemm_kernel<split>");
}

extern "C" int64_t msst_mask_estimator_workspace(const msst_band_config* c, int64_t rows) {
    BandPlan h;
    if (fill_plan(c, h) != MSST_OK || rows < 0) return -1;
    const int64_t xh = (rows * h.nb * h.dim * 2 + 255) / 256 * 256;
    const int64_t hb = (rows * h.nb * (int64_t)h.hid * 2 + 255) / 256 * 256;
    return xh + (h.L > 2 ? 2 : h.L > 1 ? 1 : 0) * hb;
}

extern "C" int msst_mask_estimator(const msst_band_config* c, const void* plan, const void* x,
                                   int x_dtype, int64_t rows, float* out, void* workspace,
                                   int64_t ws_bytes, void* stream) {
    BandPlan h;
    int rc = fill_plan(c, h);
    if (rc != MSST_OK) return rc;
    MSST_REQUIRE(plan && x && out && workspace, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(x_dtype == MSST_F32 || x_dtype == MSST_F16, MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(rows >= 0 && rows < (1 << 24), MSST_ERR_UNSUPPORTED, "rows out of range");
    MSST_REQUIRE(ws_bytes >= msst_mask_estimator_workspace(c, rows), MSST_ERR_WORKSPACE,
                 "workspace too small");
    MSST_REQUIRE(rows * h.nb * (int64_t)std::max(h.dim, h.hid) * 2 < ((int64_t)1 << 31),
                 MSST_ERR_UNSUPPORTED, "activations exceed 2^31 bytes");
    MSST_REQUIRE(aligned(x, 16) && aligned(out, 8) && aligned(workspace, 256), MSST_ERR_ALIGNMENT,
                 "x 16-byte, out 8-byte, workspace 256-byte aligned");
    if (rows == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const BandPlan* p = reinterpret_cast<const BandPlan*>(plan);
    char* ws = reinterpret_cast<char*>(workspace);
    const int64_t xh_bytes = (rows * h.nb * h.dim * 2 + 255) / 256 * 256;
    const int64_t hb_bytes = (rows * h.nb * (int64_t)h.hid * 2 + 255) / 256 * 256;
    const half_t* xh = reinterpret_cast<const half_t*>(x);
    if (x_dtype == MSST_F32) {
        // ops::linear casts its fp32 input to fp16 (ops_linear.cu:155).
        rc = msst_cast(x, MSST_F32, ws, MSST_F16, rows * h.nb * h.dim, stream);
        if (rc != MSST_OK) return rc;
        xh = reinterpret_cast<const half_t*>(ws);
    }
    half_t* hbuf[2] = {reinterpret_cast<half_t*>(ws + xh_bytes),
                       reinterpret_cast<half_t*>(ws + xh_bytes + hb_bytes)};
    const int tiles_m = (int)((rows + kBM - 1) / kBM);
    const half_t* a_cur = xh;
    int lda = h.nb * h.dim, a_band = h.dim, K = h.dim;
    int64_t a_bytes = rows * h.nb * h.dim * 2;
    for (int l = 0; l < h.L; ++l) {
        BandGemmArgs a{};
        a.plan = p;
        a.a = a_cur;
        a.a_bytes = (int)a_bytes;
        a.lda = lda;
        a.a_band = a_band;
        a.K = K;
        a.layer = l;
        a.M = (int)rows;
        a.tiles_m = tiles_m;
        if (l < h.L - 1) {
            // Hidden layer: tanh(A . W^T + b) -> [band][row][hid] fp16.
            half_t* o = hbuf[l & 1];
            a.out = o;
            a.ldo = h.hid;
            a.o_band = (int)(rows * h.hid);
            const int tiles = h.nb * tiles_m * ((h.hid + kBN - 1) / kBN);
            a.per_xcd = (tiles + 7) / 8;
            hipLaunchKernelGGL(band_gemm_kernel<kHidden>, dim3((unsigned)(8 * a.per_xcd)),
                               dim3(kGemmThreads), 0, s, a);
            rc = check_launch("band_gemm_kernel<hidden>");
            if (rc != MSST_OK) return rc;
            a_cur = o;
            lda = h.hid;
            a_band = (int)(rows * h.hid);
            K = h.hid;
            a_bytes = rows * h.nb * (int64_t)h.hid * 2;
        } else {
            // Output layer + GLU -> out [row][ftot] fp32.
            a.out = out;
            a.ldo = h.ftot;
            int tiles = 0;
            for (int b = 0; b < h.nb; ++b) tiles += tiles_m * ((2 * h.fd[b] + kBN - 1) / kBN);
            a.per_xcd = (tiles + 7) / 8;
            hipLaunchKernelGGL(band_gemm_kernel<kGlu>, dim3((unsigned)(8 * a.per_xcd)),
                               dim3(kGemmThreads), 0, s, a);
            rc = check_launch("band_gemm_kernel<glu>");
            if (rc != MSST_OK) return rc;
        }
    }
    return MSST_OK;
}

extern "C" int msst_band_gather(const msst_band_config* c, const void* plan, const float* stft,
                                int64_t batch, int64_t frames, float* out, void* stream) {
    BandPlan h;
    int rc = fill_plan(c, h);
    if (rc != MSST_OK) return rc;
    MSST_REQUIRE(h.nbins > 0, MSST_ERR_INVALID_ARG, "config has no STFT side");
    MSST_REQUIRE(plan && stft && out, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(batch >= 0 && frames >= 0 && batch < 65536 && frames < (1 << 24),
                 MSST_ERR_UNSUPPORTED, "batch / frames out of range");
    MSST_REQUIRE(aligned(stft, 8) && aligned(out, 8), MSST_ERR_ALIGNMENT, "8-byte alignment");
    if (batch == 0 || frames == 0) return MSST_OK;
    const dim3 grid((unsigned)((frames + kTile - 1) / kTile), (unsigned)((h.n_idx + kTile - 1) / kTile),
                    (unsigned)batch);
    hipLaunchKernelGGL(band_gather_kernel, grid, dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const BandPlan*>(plan), reinterpret_cast<const float2*>(stft),
                       (int)frames, reinterpret_cast<float2*>(out));
    return check_launch("band_gather_kernel");
}

extern "C" int64_t msst_mask_merge_workspace(const msst_band_config* c, int64_t batch,
                                             int64_t stems, int64_t frames) {
    BandPlan h;
    if (fill_plan(c, h) != MSST_OK || batch < 0 || stems < 0 || frames < 0) return -1;
    return h.identity ? 0 : batch * stems * frames * (int64_t)h.nbins * 8;
}

extern "C" int msst_mask_merge(const msst_band_config* c, const void* plan, const float* masks,
                               int64_t stems, const float* stft, int64_t batch, int64_t frames,
                               int zero_dc, float* out, void* workspace, int64_t ws_bytes,
                               void* stream) {
    BandPlan h;
    int rc = fill_plan(c, h);
    if (rc != MSST_OK) return rc;
    MSST_REQUIRE(h.nbins > 0, MSST_ERR_INVALID_ARG, "config has no STFT side");
    MSST_REQUIRE(plan && masks && stft && out, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(batch >= 0 && stems >= 0 && frames >= 0 && batch * stems < 65536 &&
                     frames < (1 << 24),
                 MSST_ERR_UNSUPPORTED, "batch / stems / frames out of range");
    MSST_REQUIRE(ws_bytes >= msst_mask_merge_workspace(c, batch, stems, frames),
                 MSST_ERR_WORKSPACE, "workspace too small");
    MSST_REQUIRE(h.identity || workspace, MSST_ERR_INVALID_ARG, "null workspace");
    MSST_REQUIRE(aligned(masks, 8) && aligned(stft, 8) && aligned(out, 8) &&
                     (h.identity || aligned(workspace, 16)),
                 MSST_ERR_ALIGNMENT, "8-byte alignment (workspace 16)");
    if (batch == 0 || stems == 0 || frames == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const BandPlan* p = reinterpret_cast<const BandPlan*>(plan);
    const float2* m = reinterpret_cast<const float2*>(masks);
    if (!h.identity) {
        float2* mg = reinterpret_cast<float2*>(workspace);
        const int64_t rows = stems * batch * frames;
        for (int64_t r0 = 0; r0 < rows; r0 += 65535) {
            const int64_t nr = std::min<int64_t>(65535, rows - r0);
            hipLaunchKernelGGL(mask_mean_kernel, dim3((unsigned)((h.nbins + 255) / 256), (unsigned)nr),
                               dim3(256), 0, s, p, m + r0 * h.n_idx, mg + r0 * h.nbins);
            rc = check_launch("mask_mean_kernel");
            if (rc != MSST_OK) return rc;
        }
        m = mg;
    }
    const dim3 grid((unsigned)((frames + kTile - 1) / kTile), (unsigned)((h.nbins + kTile - 1) / kTile),
                    (unsigned)(stems * batch));
    hipLaunchKernelGGL(mask_apply_kernel, grid, dim3(256), 0, s, p, m,
                       reinterpret_cast<const float2*>(stft), (int)batch, (int)frames, zero_dc,
                       reinterpret_cast<float2*>(out));
    return check_launch("mask_apply_kernel");
}
