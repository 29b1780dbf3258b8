// attention.hip — flash attention for the Roformer layers (head dim 64).
//
// Replaces the materialised pipeline of ops_attention.cu:96-181 (QK^T GEMM,
// fp32 score tensor, softmax kernel :390-452, PV GEMM) and, for the fused
// Roformer path, the surrounding head split, RoPE, gate and head merge of
// model_bs_roformer.cu:250-278 / model_mel_band_roformer.cu:34-163.  No
// N x N score tensor is ever written: scores live in MFMA accumulators and
// an online softmax (running max / running sum per query) folds each
// 64-key block into the output.
//
// Per wave: 64 queries as two 32-query MFMA column blocks.
//   S^T[key, q]  = K . Q^T     A = K from LDS, B = Q^T held in registers.
//                              Each lane owns ONE query column, so the
//                              per-query max and sum need only one
//                              cross-lane step (lane ^ 32).
//   O^T[d, q]   += V^T . P^T   A = V^T from LDS, B = P^T taken straight
//                              from the S accumulator registers — P never
//                              goes through LDS.  The rescale of O by
//                              exp2(m_old - m_new) is per lane.
// fp16 path: v_mfma_f32_32x32x16_f16.  The 8 keys a lane feeds per MFMA are
// {4h..4h+3, 8+4h..8+4h+3} of a 16-key group (that is what the S
// accumulator layout hands it); V^T is stored in LDS with key bits 2 and 3
// swapped so those 8 keys are one aligned 16-byte read.
// fp32 path: v_mfma_f32_32x32x2_f32, V in natural [key][d] layout (one key
// per lane per MFMA, so no transpose is needed).
//
// Work split: HPW (heads per workgroup) = 1 for long sequences — the 4
// waves take 4 consecutive 64-query tiles of one (sequence, head) and share
// double-buffered K/V blocks; HPW = 4 for sequences of <= 64 positions —
// each wave owns one head of the sequence.  Workgroup ids are dealt
// XCD-aware (work_item) so the query tiles of one head share an L2, with
// mostly idle last q-tiles dispatched after all full ones.
//
// RoPE (ops_misc.cu:39-69, interleaved pairs) is applied in fp32 while Q and
// K are staged; the gate (ops_fused.cu:285-303 output) multiplies the
// normalised output in the epilogue, which writes merged rows
// out[token, h*64 + d] directly.
#include <type_traits>

#include "msst_common.hpp"

namespace msst {
namespace {

constexpr int kD = 64;
constexpr int kKB = 64;  // keys per block

struct AttnParams {
    const void* q;
    const void* k;
    const void* v;
    void* out;
    int64_t ld_in, ld_out;      // token row strides (elements)
    int64_t head_in, head_out;  // element offset of head h within a row
    const float* cos_t;         // [N, 32] or null
    const float* sin_t;
    const float* gates;         // [token, H] or null
    int64_t n_inner;
    int64_t q_outer, q_inner, q_pos;
    int64_t k_outer, k_inner, k_pos;
    int n_q, n_k;               // queries / keys per sequence
    int H;
    int qtiles;                 // q-tiles per (seq, head): waves_per_head x 64 queries (x 32: fp32, one head)
    int64_t total_items;        // workgroup work items
    int per_xcd;                // work items per XCD (see work_item)
    int short_last;             // most waves of a pair's last q-tile are idle
    float scale_log2;           // softmax scale * log2(e)
};

__device__ __forceinline__ int64_t tok_q(const AttnParams& p, int64_t s, int64_t pos) {
    return (s / p.n_inner) * p.q_outer + (s % p.n_inner) * p.q_inner + pos * p.q_pos;
}
__device__ __forceinline__ int64_t tok_k(const AttnParams& p, int64_t s, int64_t pos) {
    return (s / p.n_inner) * p.k_outer + (s % p.n_inner) * p.k_inner + pos * p.k_pos;
}

// Rotate the 4 interleaved pairs held in x[0..7] (head dims 2i..2i+7,
// pair index pi0 .. pi0+3) by the angles of position pos.
__device__ __forceinline__ void rope8(float (&x)[8], const float* cos_t, const float* sin_t,
                                      int pos, int pi0) {
    f4 c = *reinterpret_cast<const f4*>(cos_t + pos * (kD / 2) + pi0);
    f4 s = *reinterpret_cast<const f4*>(sin_t + pos * (kD / 2) + pi0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float a = x[2 * e], b = x[2 * e + 1];
        x[2 * e] = a * c[e] - b * s[e];
        x[2 * e + 1] = a * s[e] + b * c[e];
    }
}

__device__ __forceinline__ int swap_bits23(int kr) {
    return (kr & ~0xC) | ((kr & 4) << 1) | ((kr & 8) >> 1);
}

// Work item of this workgroup: (sequence, head group) pair sh and q-tile
// qt.  Workgroups are dealt round-robin to the 8 XCDs (workgroup b runs on
// XCD b % 8), so XCD x is given a contiguous run of the items and walks it
// in dispatch order b / 8; the q-tiles of one pair are adjacent, so they
// run together and share K/V in that XCD's L2.  When most waves of the last
// q-tile of a pair are idle (p.short_last), XCD x is given the pairs
// [x per, x per + per) and walks first every q-tile but the last of each
// pair, then the last q-tile of each: the short workgroups fill the end of
// the grid instead of holding workgroup slots beside full ones.  Returns
// false for the grid's padding workgroups.
__device__ __forceinline__ bool work_item(const AttnParams& p, int64_t& sh, int& qt) {
    const int64_t b = blockIdx.x;
    const int64_t l = b >> 3;
    const int Q = p.qtiles;
    if (!p.short_last) {
        const int64_t item = (b & 7) * (int64_t)p.per_xcd + l;
        if (item >= p.total_items) return false;
        sh = item / Q;
        qt = (int)(item % Q);
        return true;
    }
    const int64_t S = p.total_items / Q;
    const int64_t per = (S + 7) / 8;
    const int64_t base = (b & 7) * per;
    const int64_t n = min(per, S - base);
    if (n <= 0) return false;
    if (l < n * (Q - 1)) {
        sh = base + l / (Q - 1);
        qt = (int)(l % (Q - 1));
    } else if (l < n * Q) {
        sh = base + (l - n * (Q - 1));
        qt = Q - 1;
    } else {
        return false;
    }
    return true;
}

// ===========================================================================
// fp16
// ===========================================================================
template <int HPW>
__global__ __launch_bounds__(256) void attn_f16_kernel(AttnParams p) {
    constexpr int WPH = 4 / HPW;          // waves per head
    constexpr int NSLOT = HPW == 1 ? 2 : 4;
    constexpr int SLOT = 2 * kKB * kD;    // K block + V^T block (halves)
    constexpr int GROUP = 256 / HPW;      // threads loading one head's block
    constexpr int CH = kKB * 8 / GROUP;   // 16-byte chunks per thread per tensor
    __shared__ __attribute__((aligned(16))) half_t lds[NSLOT * SLOT];

    int64_t sh;
    int qt_idx;
    if (!work_item(p, sh, qt_idx)) return;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lrow = lane & 31, lh = lane >> 5;
    const int head_local = w / WPH, qsub = w % WPH;
    const int head_groups = (p.H + HPW - 1) / HPW;
    const int hg = (int)(sh % head_groups);
    const int64_t seq = sh / head_groups;
    const int h = hg * HPW + head_local;
    const bool head_ok = h < p.H;
    const int q0 = (qt_idx * WPH + qsub) * 64;
    const bool wave_active = head_ok && q0 < p.n_q;

    const half_t* qb = reinterpret_cast<const half_t*>(p.q);
    const half_t* kbp = reinterpret_cast<const half_t*>(p.k);
    const half_t* vbp = reinterpret_cast<const half_t*>(p.v);

    // ---- Q operand (B of S^T = K . Q^T), RoPE applied, held for the loop.
    h8 qf[2][4];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const bool ok = wave_active && qi < p.n_q;
        const half_t* row = qb + (ok ? tok_q(p, seq, qi) * p.ld_in + h * p.head_in : 0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const int d0 = kk * 16 + lh * 8;
            if (ok) {
                h8 raw = *reinterpret_cast<const h8*>(row + d0);
                if (p.cos_t) {
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = (float)raw[e];
                    rope8(x, p.cos_t, p.sin_t, qi, d0 / 2);
#pragma unroll
                    for (int e = 0; e < 8; ++e) raw[e] = (half_t)x[e];
                }
                qf[qt][kk] = raw;
            } else {
                qf[qt][kk] = h8{};
            }
        }
    }

    // ---- K/V block staging: this thread's group loads head h_load.
    const int grp = tid / GROUP, gt = tid % GROUP;
    const int h_load = hg * HPW + grp;
    const bool load_ok = h_load < p.H;
    h8 kreg[CH], vreg[CH];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int chunk = gt + i * GROUP;  // 0..511
            const int kr = chunk >> 3, c = chunk & 7;
            const int key = kb * kKB + kr;
            if (load_ok && key < p.n_k) {
                const int64_t off = tok_k(p, seq, key) * p.ld_in + h_load * p.head_in + c * 8;
                h8 kv = *reinterpret_cast<const h8*>(kbp + off);
                if (p.cos_t) {
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) x[e] = (float)kv[e];
                    rope8(x, p.cos_t, p.sin_t, key, c * 4);
#pragma unroll
                    for (int e = 0; e < 8; ++e) kv[e] = (half_t)x[e];
                }
                kreg[i] = kv;
                vreg[i] = *reinterpret_cast<const h8*>(vbp + off);
            } else {
                kreg[i] = h8{};
                vreg[i] = h8{};  // zero V rows: masked keys contribute 0 * 0
            }
        }
    };
    auto store_block = [&](int slot) {
        half_t* Ks = lds + slot * SLOT;
        half_t* Vt = Ks + kKB * kD;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int chunk = gt + i * GROUP;
            const int kr = chunk >> 3, c = chunk & 7;
            *reinterpret_cast<h8*>(Ks + kr * kD + ((c ^ (kr & 7)) << 3)) = kreg[i];
            const int pos = swap_bits23(kr);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int d = c * 8 + e;
                const int sw = (d ^ (d >> 3)) & 7;
                Vt[d * kKB + ((((pos >> 3) ^ sw)) << 3) + (pos & 7)] = vreg[i][e];
            }
        }
    };

    f16x o[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) o[a][b] = f16x{};
    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.0f, 0.0f};

    const int nkb = (p.n_k + kKB - 1) / kKB;
    const int my_slot0 = HPW == 1 ? 0 : grp;
    load_block(0);
    store_block(my_slot0);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const int slot = HPW == 1 ? (kb & 1) : head_local;
        if (HPW == 1 && kb + 1 < nkb) load_block(kb + 1);
        if (wave_active) {
            const half_t* Ks = lds + slot * SLOT;
            const half_t* Vt = Ks + kKB * kD;
            // S^T for the two 32-key halves and the two query blocks.
            f16x s[2][2];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
                s[k2][0] = f16x{};
                s[k2][1] = f16x{};
                const int kr = k2 * 32 + lrow;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const int c = kk * 2 + lh;
                    h8 kf = *reinterpret_cast<const h8*>(Ks + kr * kD + ((c ^ (kr & 7)) << 3));
                    s[k2][0] = mfma32x32x16(kf, qf[0][kk], s[k2][0]);
                    s[k2][1] = mfma32x32x16(kf, qf[1][kk], s[k2][1]);
                }
            }
            const int key_base = kb * kKB;
            const bool tail = key_base + kKB > p.n_k;
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                float mx = -INFINITY;
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        float x = s[k2][qt][v] * p.scale_log2;
                        if (tail) {
                            const int key = key_base + k2 * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                            if (key >= p.n_k) x = -INFINITY;
                        }
                        s[k2][qt][v] = x;
                        mx = fmaxf(mx, x);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float m_new = fmaxf(m_run[qt], mx);
                const float alpha = exp2f(m_run[qt] - m_new);
                m_run[qt] = m_new;
                float psum = 0.0f;
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        float e = exp2f(s[k2][qt][v] - m_new);
                        s[k2][qt][v] = e;
                        psum += e;
                    }
                l_run[qt] = l_run[qt] * alpha + psum;
#pragma unroll
                for (int dm = 0; dm < 2; ++dm)
#pragma unroll
                    for (int v = 0; v < 16; ++v) o[qt][dm][v] *= alpha;
            }
            // O^T += V^T . P^T over 4 sixteen-key substeps.
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const int k2 = t >> 1, tp = t & 1;
                h8 pf[2];
#pragma unroll
                for (int qt = 0; qt < 2; ++qt)
#pragma unroll
                    for (int e = 0; e < 8; ++e) pf[qt][e] = (half_t)s[k2][qt][8 * tp + e];
                const int chunk = k2 * 4 + 2 * tp + lh;
#pragma unroll
                for (int dm = 0; dm < 2; ++dm) {
                    const int d = dm * 32 + lrow;
                    const int sw = (d ^ (d >> 3)) & 7;
                    h8 vf = *reinterpret_cast<const h8*>(Vt + d * kKB + ((chunk ^ sw) << 3));
                    o[0][dm] = mfma32x32x16(vf, pf[0], o[0][dm]);
                    o[1][dm] = mfma32x32x16(vf, pf[1], o[1][dm]);
                }
            }
        }
        if (HPW == 1 && kb + 1 < nkb) store_block((kb + 1) & 1);
        __syncthreads();
    }

    if (!wave_active) return;
    half_t* ob = reinterpret_cast<half_t*>(p.out);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const float l_tot = l_run[qt] + __shfl_xor(l_run[qt], 32, 64);
        if (qi >= p.n_q) continue;
        const int64_t tok = tok_q(p, seq, qi);
        float scale = 1.0f / l_tot;
        if (p.gates) scale *= p.gates[tok * p.H + h];
        half_t* orow = ob + tok * p.ld_out + h * p.head_out;
#pragma unroll
        for (int dm = 0; dm < 2; ++dm)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = dm * 32 + 8 * g + 4 * lh;
                h4 val;
#pragma unroll
                for (int e = 0; e < 4; ++e) val[e] = (half_t)(o[qt][dm][4 * g + e] * scale);
                *reinterpret_cast<h4*>(orow + d) = val;
            }
    }
}

// ===========================================================================
// fp16 with q/k already rotated (no RoPE tables): K and V by LDS DMA
// ===========================================================================
// Each 64-key block lands in LDS as two [64 rows][128 B] tiles in token
// layout, written by buffer_load ... lds (no VGPR staging, no VALU).
//   K fragments (A of S^T = K . Q^T) are 16-byte row reads; chunk c of row r
//   sits at c ^ ((r >> 1) & 7), so the 16 rows one b128 pass serves hit
//   distinct banks.
//   V^T fragments (A of O^T += V^T . P^T) come from ds_read_b64_tr_b16:
//   within each 16-lane group, output lane j element e is element j % 4 of
//   the 8 bytes read by lane 4e + j / 4.  Lane s of the group points at row
//   key0 + s / 4, columns d0 + 4 (s % 4) .. + 3, so lane j receives keys
//   key0 .. key0 + 3 of column d0 + j: the transposed fragment, straight
//   from the token-layout tile.  Chunk c of V row r sits at
//   c ^ (4 ((r >> 1) & 1)): the 4 rows x 4 chunks of one half-wave read
//   then map to distinct banks.
// Softmax: the score scale folds into the FMA feeding v_exp_f32
// (s * c - m * c, c = scale * log2 e).  The running max only moves when a
// half-block's max exceeds it by more than 8 (log2 units): most half-blocks
// skip the rescale of O, and P stays <= 2^8 (exact range for fp16).  Row
// sums add the fp16 P values the PV MFMA consumes (v_dot2 against 1.0), so
// numerator and denominator see the same rounding.  The lane ^ 32 partner
// of a query's scores is reached with v_permlane32_swap.
// Schedule: a 64-key block is two 32-key halves, each run S -> softmax ->
// PV in turn, so only one half's scores and P are live: the HPW = 1 kernel
// fits 168 VGPRs and runs three workgroups (12 waves) per CU, whose waves
// overlap one another's MFMA and VALU phases.  (Issuing S of half 1 ahead
// of half 0's softmax, for overlap within a wave, needed ~200 VGPRs, two
// workgroups per CU, and ran 9-15 % slower.)
// HPW = 1: 4 waves x 64 queries of one (sequence, head) share a 3-stage K/V
// ring (each wave DMAs 16 of the 64 rows; fence-free barrier; the next two
// blocks in flight while a block computes).  HPW = 4 (<= 64 keys):
// each wave owns one head and DMAs its own single block.
typedef short s4_t __attribute__((__vector_size__(4 * sizeof(short))));
typedef __attribute__((address_space(3))) s4_t lds_s4_t;

__device__ __forceinline__ h4 lds_read_tr16(const lds_half_t* ptr) {
    const s4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(ptr));
    return __builtin_bit_cast(h4, v);
}

// V^T fragment reads for the unrolled K/V ring, as inline asm.  The
// compiler treats any LDS read it can see as possibly aliasing the ring's
// in-flight LDS DMAs and waits for all of them (vmcnt(0)) first, which
// would wait for the block prefetched two blocks ahead.  So the reads are
// issued by asm (invisible to that analysis) and completed by an asm
// lgkmcnt wait tied to their registers, so no user is scheduled above it.
//
// Issue (no wait) the four transposed reads of two V^T fragments at
// a0 + OFF and a1 + OFF (rows r and r + 8 each).
template <int OFF>
__device__ __forceinline__ void lds_read_tr16_issue4(uint32_t a0, uint32_t a1, s4_t (&r)[4]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %4 offset:%6\n\t"
        "ds_read_b64_tr_b16 %1, %4 offset:%7\n\t"
        "ds_read_b64_tr_b16 %2, %5 offset:%6\n\t"
        "ds_read_b64_tr_b16 %3, %5 offset:%7"
        : "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3])
        : "v"(a0), "v"(a1), "n"(OFF), "n"(OFF + 8 * kD * 2));
}
// Wait until at most N LDS operations are outstanding.  LDS operations
// complete in issue order, and any other LDS or scalar-memory operation the
// compiler issues in between only adds to the count, so with N = the reads
// issued after those needed, the wait can only be stricter than required.
// The registers are tied to the wait so their users cannot move above it.
template <int N>
__device__ __forceinline__ void lds_wait_tied(s4_t (&r)[4]) {
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]) : "n"(N));
}
__device__ __forceinline__ h8 cat_h8(const s4_t& lo, const s4_t& hi) {
    return __builtin_shufflevector(__builtin_bit_cast(h4, lo), __builtin_bit_cast(h4, hi), 0, 1, 2,
                                   3, 4, 5, 6, 7);
}

// Maxima of scores: llvm.maximum, which gfx950 lowers to v_maximum3_f32
// / v_maximum_f32 (NaN-propagating) with no input canonicalisation, where
// fmaxf in IEEE mode would first quiet every input with an extra
// v_max x, x.  Being compiler-visible (not inline asm), these reads of MFMA
// accumulators get the MFMA-to-VALU wait states from the compiler's hazard
// tracking, which does not look inside inline asm.
__device__ __forceinline__ float fmax_nc(float a, float b) {
    return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float fmax3_nc(float a, float b, float c) {
    return fmax_nc(fmax_nc(a, b), c);
}

// max over the query's two lanes (l, l ^ 32).
__device__ __forceinline__ float pair_max(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false,
                                                    false);
    return fmax_nc(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float a) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

constexpr float kRescaleLog2 = 8.0f;

template <int HPW>
constexpr int dma_nslot() { return HPW == 1 ? 3 : 4; }

// One work item of attn_f16_dma_kernel.  QT: 32-query column blocks per wave
// (2: 64 queries per wave; 1: the tail q-tile of a sequence, 16 queries per
// wave, so its rows are spread over the workgroup's waves).
template <int HPW, int QT>
__device__ __forceinline__ void attn_dma_item(const AttnParams& p, int64_t sh, int qt_idx,
                                              half_t* lds) {
    constexpr int WPH = 4 / HPW;
    constexpr int NSLOT = dma_nslot<HPW>();
    constexpr int SLOT = 2 * kKB * kD;          // halves: K tile, then V tile
    constexpr int ROWS_W = HPW == 1 ? 16 : 64;  // block rows one wave DMAs
    constexpr int NDMA = 2 * ROWS_W / 8;        // DMA instructions per wave per block
    constexpr int QROWS = QT == 2 ? 64 : 16;    // queries per wave
    static_assert(QT == 2 || HPW == 1, "tail q-tiles are split only in the one-head form");

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 31, lh = lane >> 5;
    const int head_local = w / WPH, qsub = w % WPH;
    const int head_groups = (p.H + HPW - 1) / HPW;
    const int hg = (int)(sh % head_groups);
    const int64_t seq = sh / head_groups;
    const int h = hg * HPW + head_local;
    const bool head_ok = h < p.H;  // always true for HPW = 1
    const int q0 = QT == 2 ? (qt_idx * WPH + qsub) * 64 : qt_idx * WPH * 64 + w * QROWS;
    const int q_end = min(q0 + QROWS, p.n_q);  // this wave's queries: [q0, q_end)
    const bool wave_active = head_ok && q0 < p.n_q;

    // ---- Q operand (B of S^T), held for the whole loop.
    const half_t* qb = reinterpret_cast<const half_t*>(p.q);
    h8 qf[QT][4];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const bool ok = wave_active && qi < q_end;
        const half_t* row = qb + (ok ? tok_q(p, seq, qi) * p.ld_in + h * p.head_in : 0);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
            qf[qt][kk] = ok ? *reinterpret_cast<const h8*>(row + kk * 16 + lh * 8) : h8{};
    }

    // ---- K/V DMA.  Rows past the sequence re-read its last key (masked in
    // the scores, and finite, so P = 0 times V adds exactly 0).
    const int64_t base_off = head_ok ? tok_k(p, seq, 0) * p.ld_in + h * p.head_in : 0;
    const half_t* kbase = uniform_ptr(reinterpret_cast<const half_t*>(p.k) + base_off);
    const half_t* vbase = uniform_ptr(reinterpret_cast<const half_t*>(p.v) + base_off);
    const uint32_t rsb = (uint32_t)(p.k_pos * p.ld_in * 2);  // bytes between keys
    const int span = (int)((p.n_k - 1) * rsb) + kD * 2;
    const int row0w = HPW == 1 ? w * ROWS_W : 0;
    const int sub = lane >> 3, pch = lane & 7;
    lds_half_t* const L = (lds_half_t*)lds;
    auto slot_ptr = [&](int kb) -> lds_half_t* {
        return L + (HPW == 1 ? (kb % NSLOT) : head_local) * SLOT;
    };
    auto issue = [&](lds_half_t* Ks, int kb) {
        lds_half_t* Vs = Ks + kKB * kD;
#pragma unroll
        for (int i = 0; i < ROWS_W / 8; ++i) {
            const int r = row0w + i * 8 + sub;
            const uint32_t ro = (uint32_t)min(kb * kKB + r, p.n_k - 1) * rsb;
            dma16(kbase, span, Ks + (row0w + i * 8) * kD, ro + ((pch ^ ((r >> 1) & 7)) << 4));
            dma16(vbase, span, Vs + (row0w + i * 8) * kD,
                  ro + ((pch ^ (((r >> 1) & 1) << 2)) << 4));
        }
    };

    // Per-lane byte offsets of the fragment reads within a slot (the XOR
    // swizzles make them lane-dependent; everything else is an immediate).
    const int kr_sw = (lrow >> 1) & 7;
    int kofs[4];  // halves
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) kofs[kk] = lrow * kD + (((kk * 2 + lh) ^ kr_sw) << 3);
    const int g = lane >> 4, j16 = lane & 15;
    const int vrow = 4 * (g >> 1) + (j16 >> 2);  // row within an 8-key group
    const int vsw = ((vrow >> 1) & 1) << 2;
    const int vch = 2 * (g & 1) + ((j16 & 3) >> 1);
    const int vsub = (j16 & 1) * 4;
    int voff[2];  // halves, from the slot start (V tile follows the K tile)
#pragma unroll
    for (int dm = 0; dm < 2; ++dm)
        voff[dm] = kKB * kD + vrow * kD + (((4 * dm + vch) ^ vsw) << 3) + vsub;

    f16x o[QT][2];
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int a = 0; a < QT; ++a) {
        o[a][0] = f16x{};
        o[a][1] = f16x{};
        m_run[a] = -INFINITY;
        l_run[a] = 0.0f;
    }
    const float c = p.scale_log2;
    const float th = kRescaleLog2 / c;
    const h2 ones = h2{(half_t)1.0f, (half_t)1.0f};

    // S^T for the 32 keys of half hf: sh[qt] (keys hf*32 + 8 (v/4) + 4 lh + v%4).
    auto s_half = [&](const lds_half_t* Ks, int hf, f16x (&shf)[QT]) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) shf[qt] = f16x{};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const h8 kf = *(const lds_h8_t*)(Ks + kofs[kk] + hf * 32 * kD);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) shf[qt] = mfma32x32x16(kf, qf[qt][kk], shf[qt]);
        }
    };
    // Online softmax of one half: P^T operands pf[qt][tp] (16-key substeps).
    auto softmax_half = [&](auto tail_c, int key0, f16x (&shf)[QT], h8 (&pf)[QT][2]) {
        constexpr bool TAIL = decltype(tail_c)::value;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            if constexpr (TAIL) {
                // Register v holds key key0 + 4 lh + 8 (v / 4) + v % 4: one
                // per-lane limit against immediates (no per-key registers).
                const int lim = p.n_k - key0 - 4 * lh;
#pragma unroll
                for (int v = 0; v < 16; ++v)
                    if (8 * (v >> 2) + (v & 3) >= lim) shf[qt][v] = -INFINITY;
            }
            float m = fmax3_nc(shf[qt][0], shf[qt][1], shf[qt][2]);
#pragma unroll
            for (int v = 3; v < 15; v += 2) m = fmax3_nc(m, shf[qt][v], shf[qt][v + 1]);
            const float mx = pair_max(fmax_nc(m, shf[qt][15]));
            if (mx > m_run[qt] + th) {
                const float alpha = __builtin_amdgcn_exp2f((m_run[qt] - mx) * c);
                m_run[qt] = mx;
                l_run[qt] *= alpha;
#pragma unroll
                for (int dm = 0; dm < 2; ++dm)
#pragma unroll
                    for (int v = 0; v < 16; ++v) o[qt][dm][v] *= alpha;
            }
            const float nmc = -m_run[qt] * c;
            float ls = 0.0f;
#pragma unroll
            for (int tp = 0; tp < 2; ++tp)
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const float p0 = __builtin_amdgcn_exp2f(fmaf(shf[qt][8 * tp + e], c, nmc));
                    const float p1 =
                        __builtin_amdgcn_exp2f(fmaf(shf[qt][8 * tp + e + 1], c, nmc));
                    const h2 pp = h2{(half_t)p0, (half_t)p1};
                    pf[qt][tp][e] = pp[0];
                    pf[qt][tp][e + 1] = pp[1];
                    ls = __builtin_amdgcn_fdot2(pp, ones, ls, false);
                }
            l_run[qt] += ls;
        }
    };
    // O^T += V^T . P^T over the two 16-key substeps of half hf.
    auto pv_half = [&](const lds_half_t* Ks, int hf, h8 (&pf)[QT][2]) {
#pragma unroll
        for (int tp = 0; tp < 2; ++tp)
#pragma unroll
            for (int dm = 0; dm < 2; ++dm) {
                const lds_half_t* vp = Ks + voff[dm] + (hf * 2 + tp) * 16 * kD;
                const h4 lo = lds_read_tr16(vp);
                const h4 hi = lds_read_tr16(vp + 8 * kD);
                const h8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) o[qt][dm] = mfma32x32x16(vf, pf[qt][tp], o[qt][dm]);
            }
    };
    // The same with the slot S and half HF known at compile time: the V^T
    // fragment reads take two per-lane base addresses and immediate offsets.
    uint32_t va[2];
#pragma unroll
    for (int dm = 0; dm < 2; ++dm) va[dm] = (uint32_t)(uintptr_t)(L + voff[dm]);
    auto pv_half_imm = [&](auto slot_c, auto hf_c, h8 (&pf)[QT][2]) __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value, HF = decltype(hf_c)::value;
        constexpr int B0 = (S * SLOT + (HF * 2 + 0) * 16 * kD) * 2;
        constexpr int B1 = (S * SLOT + (HF * 2 + 1) * 16 * kD) * 2;
        s4_t r0[4], r1[4];
        lds_read_tr16_issue4<B0>(va[0], va[1], r0);
        lds_read_tr16_issue4<B1>(va[0], va[1], r1);
        lds_wait_tied<4>(r0);
        const h8 v00 = cat_h8(r0[0], r0[1]), v01 = cat_h8(r0[2], r0[3]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][0] = mfma32x32x16(v00, pf[qt][0], o[qt][0]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][1] = mfma32x32x16(v01, pf[qt][0], o[qt][1]);
        lds_wait_tied<0>(r1);
        const h8 v10 = cat_h8(r1[0], r1[1]), v11 = cat_h8(r1[2], r1[3]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][0] = mfma32x32x16(v10, pf[qt][1], o[qt][0]);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) o[qt][1] = mfma32x32x16(v11, pf[qt][1], o[qt][1]);
    };
    // slot_c: the ring slot as a compile-time constant, or -1 for a slot
    // known only at run time (Ks).
    auto block = [&](auto tail_c, auto slot_c, const lds_half_t* Ks, int key_base)
                     __attribute__((always_inline)) {
        constexpr int S = decltype(slot_c)::value;
        f16x sa[QT], sb[QT];
        h8 pa[QT][2], pb[QT][2];
        s_half(Ks, 0, sa);
        softmax_half(tail_c, key_base, sa, pa);
        if constexpr (S >= 0)
            pv_half_imm(slot_c, std::integral_constant<int, 0>{}, pa);
        else
            pv_half(Ks, 0, pa);
        s_half(Ks, 1, sb);
        softmax_half(tail_c, key_base + 32, sb, pb);
        if constexpr (S >= 0)
            pv_half_imm(slot_c, std::integral_constant<int, 1>{}, pb);
        else
            pv_half(Ks, 1, pb);
    };
    using runtime_slot = std::integral_constant<int, -1>;

    const int nkb = (p.n_k + kKB - 1) / kKB;
    if constexpr (HPW == 1) {
        // 3-stage ring: blocks kb and kb + 1 in flight before block kb is used.
        // The loop is unrolled by the ring's three slots, so every LDS
        // address is a lane offset plus an immediate (a runtime slot index
        // costs a VALU add per fragment address).
        auto step = [&](auto slot_c, int kb) __attribute__((always_inline)) {
            constexpr int S = decltype(slot_c)::value;
            if (kb + 1 < nkb)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NDMA) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            // Block kb has landed for every wave; slot (kb + 2) % 3 was last
            // read in iteration kb - 1, which every wave has finished.
            lds_barrier();
            if (kb + 2 < nkb) issue(L + ((S + 2) % NSLOT) * SLOT, kb + 2);
            // Full blocks only here; a partial last block is peeled below so
            // the masking code does not share this loop's registers.
            if (wave_active && (kb + 1) * kKB <= p.n_k) block(std::false_type{}, slot_c, L + S * SLOT, kb * kKB);
        };
        issue(L, 0);
        if (nkb > 1) issue(L + SLOT, 1);
        for (int kb = 0; kb < nkb; kb += NSLOT) {
            step(std::integral_constant<int, 0>{}, kb);
            if (kb + 1 < nkb) step(std::integral_constant<int, 1>{}, kb + 1);
            if (kb + 2 < nkb) step(std::integral_constant<int, 2>{}, kb + 2);
        }
        if (wave_active && nkb * kKB > p.n_k)
            block(std::true_type{}, runtime_slot{}, slot_ptr(nkb - 1), (nkb - 1) * kKB);
    } else {
        // One block per wave, in the wave's own slot: the host selects this
        // variant only for sequences of at most 64 keys (launch_attention).
        if (head_ok) issue(slot_ptr(0), 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        lds_barrier();
        if (wave_active) {
            if (p.n_k < kKB)
                block(std::true_type{}, runtime_slot{}, slot_ptr(0), 0);
            else
                block(std::false_type{}, runtime_slot{}, slot_ptr(0), 0);
        }
    }

    if (!wave_active) return;
    half_t* ob = reinterpret_cast<half_t*>(p.out);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const float l_tot = pair_sum(l_run[qt]);
        if (qi >= q_end) continue;
        const int64_t tok = tok_q(p, seq, qi);
        float scale = 1.0f / l_tot;
        if (p.gates) scale *= p.gates[tok * p.H + h];
        half_t* orow = ob + tok * p.ld_out + h * p.head_out;
#pragma unroll
        for (int dm = 0; dm < 2; ++dm)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) {
                const int d = dm * 32 + 8 * gg + 4 * lh;
                h4 val;
#pragma unroll
                for (int e = 0; e < 4; ++e) val[e] = (half_t)(o[qt][dm][4 * gg + e] * scale);
                *reinterpret_cast<h4*>(orow + d) = val;
            }
    }
}

template <int HPW>
__global__ __launch_bounds__(256, HPW == 1 ? 3 : 2) void attn_f16_dma_kernel(AttnParams p) {
    __shared__ __attribute__((aligned(16))) half_t lds[dma_nslot<HPW>() * 2 * kKB * kD];
    int64_t sh;
    int qt_idx;
    if (!work_item(p, sh, qt_idx)) return;
    if constexpr (HPW == 1) {
        // The tail q-tile of a sequence with at most 64 queries left would
        // run one wave of four for the full key loop; its rows go 16 per wave
        // instead (one 32-query column block each: half a wave's MFMA work).
        if (qt_idx == p.qtiles - 1 && p.n_q - qt_idx * 256 <= 64) {
            attn_dma_item<1, 1>(p, sh, qt_idx, lds);
            return;
        }
    }
    attn_dma_item<HPW, 2>(p, sh, qt_idx, lds);
}

// ===========================================================================
// fp32
// ===========================================================================
template <int HPW, int QT>
__global__ __launch_bounds__(256, QT == 1 ? 2 : 1) void attn_f32_kernel(AttnParams p) {
    constexpr int WPH = 4 / HPW;
    constexpr int SLOT = 2 * kKB * kD;   // K block + V block (floats)
    constexpr int GROUP = 256 / HPW;
    constexpr int CH = kKB * 16 / GROUP;  // 16-byte chunks (4 floats) per thread
    extern __shared__ __attribute__((aligned(16))) float lds_f[];

    int64_t sh;
    int qt_idx;
    if (!work_item(p, sh, qt_idx)) return;

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lrow = lane & 31, lh = lane >> 5;
    const int head_local = w / WPH, qsub = w % WPH;
    const int head_groups = (p.H + HPW - 1) / HPW;
    const int hg = (int)(sh % head_groups);
    const int64_t seq = sh / head_groups;
    const int h = hg * HPW + head_local;
    const bool head_ok = h < p.H;
    const int q0 = (qt_idx * WPH + qsub) * 32 * QT;
    const bool wave_active = head_ok && q0 < p.n_q;

    const float* qb = reinterpret_cast<const float*>(p.q);
    const float* kbp = reinterpret_cast<const float*>(p.k);
    const float* vbp = reinterpret_cast<const float*>(p.v);

    // Q operand: lane (query, half h) holds Q[q][32h .. 32h+31].
    float qf[QT][32];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const bool ok = wave_active && qi < p.n_q;
        const float* row = qb + (ok ? tok_q(p, seq, qi) * p.ld_in + h * p.head_in : 0);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float x[8];
            if (ok) {
                f4 a = *reinterpret_cast<const f4*>(row + 32 * lh + 8 * c);
                f4 b = *reinterpret_cast<const f4*>(row + 32 * lh + 8 * c + 4);
                x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3];
                x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
                if (p.cos_t) rope8(x, p.cos_t, p.sin_t, qi, 16 * lh + 4 * c);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.0f;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) qf[qt][8 * c + e] = x[e];
        }
    }

    const int grp = tid / GROUP, gt = tid % GROUP;
    const int h_load = hg * HPW + grp;
    const bool load_ok = h_load < p.H;
    f4 kreg[CH], vreg[CH];
    auto load_block = [&](int kb) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int chunk = gt + i * GROUP;  // 0..1023
            const int kr = chunk >> 4, c = chunk & 15;
            const int key = kb * kKB + kr;
            if (load_ok && key < p.n_k) {
                const int64_t off = tok_k(p, seq, key) * p.ld_in + h_load * p.head_in + c * 4;
                f4 kv = *reinterpret_cast<const f4*>(kbp + off);
                if (p.cos_t) {
                    // dims 4c..4c+3 are the pairs 2c and 2c+1
                    const float* ct = p.cos_t + key * (kD / 2) + c * 2;
                    const float* st = p.sin_t + key * (kD / 2) + c * 2;
                    const float c0 = ct[0], c1 = ct[1], s0 = st[0], s1 = st[1];
                    float a0 = kv[0], b0 = kv[1], a1 = kv[2], b1 = kv[3];
                    kv[0] = a0 * c0 - b0 * s0;
                    kv[1] = a0 * s0 + b0 * c0;
                    kv[2] = a1 * c1 - b1 * s1;
                    kv[3] = a1 * s1 + b1 * c1;
                }
                kreg[i] = kv;
                vreg[i] = *reinterpret_cast<const f4*>(vbp + off);
            } else {
                kreg[i] = f4{};
                vreg[i] = f4{};
            }
        }
    };
    auto store_block = [&](int slot) {
        float* Ks = lds_f + slot * SLOT;
        float* Vs = Ks + kKB * kD;
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const int chunk = gt + i * GROUP;
            const int kr = chunk >> 4, c = chunk & 15;
            *reinterpret_cast<f4*>(Ks + kr * kD + ((c ^ (kr & 15)) << 2)) = kreg[i];
            *reinterpret_cast<f4*>(Vs + kr * kD + (c << 2)) = vreg[i];
        }
    };

    f16x o[QT][2];
#pragma unroll
    for (int a = 0; a < QT; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) o[a][b] = f16x{};
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int a = 0; a < QT; ++a) {
        m_run[a] = -INFINITY;
        l_run[a] = 0.0f;
    }

    const int nkb = (p.n_k + kKB - 1) / kKB;
    load_block(0);
    store_block(HPW == 1 ? 0 : grp);
    __syncthreads();

    for (int kb = 0; kb < nkb; ++kb) {
        const int slot = HPW == 1 ? (kb & 1) : head_local;
        if (HPW == 1 && kb + 1 < nkb) load_block(kb + 1);
        if (wave_active) {
            const float* Ks = lds_f + slot * SLOT;
            const float* Vs = Ks + kKB * kD;
            f16x s[2][QT];
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) s[k2][qt] = f16x{};
                const int kr = k2 * 32 + lrow;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const int cc = 8 * lh + c;  // K dims 32h + 4c .. +3
                    f4 kf = *reinterpret_cast<const f4*>(Ks + kr * kD + ((cc ^ (kr & 15)) << 2));
#pragma unroll
                    for (int e = 0; e < 4; ++e)
#pragma unroll
                        for (int qt = 0; qt < QT; ++qt)
                            s[k2][qt] = mfma32x32x2f32(kf[e], qf[qt][4 * c + e], s[k2][qt]);
                }
            }
            const int key_base = kb * kKB;
            const bool tail = key_base + kKB > p.n_k;
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                float mx = -INFINITY;
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        float x = s[k2][qt][v] * p.scale_log2;
                        if (tail) {
                            const int key = key_base + k2 * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
                            if (key >= p.n_k) x = -INFINITY;
                        }
                        s[k2][qt][v] = x;
                        mx = fmaxf(mx, x);
                    }
                mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
                const float m_new = fmaxf(m_run[qt], mx);
                const float alpha = exp2f(m_run[qt] - m_new);
                m_run[qt] = m_new;
                float psum = 0.0f;
#pragma unroll
                for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                    for (int v = 0; v < 16; ++v) {
                        float e = exp2f(s[k2][qt][v] - m_new);
                        s[k2][qt][v] = e;
                        psum += e;
                    }
                l_run[qt] = l_run[qt] * alpha + psum;
#pragma unroll
                for (int dm = 0; dm < 2; ++dm)
#pragma unroll
                    for (int v = 0; v < 16; ++v) o[qt][dm][v] *= alpha;
            }
            // O^T += V^T . P^T: substep v of key half k2 feeds key
            // k2*32 + 8(v/4) + 4h + v%4, which is register v of S.
#pragma unroll
            for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int key = k2 * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
#pragma unroll
                    for (int dm = 0; dm < 2; ++dm) {
                        const float vf = Vs[key * kD + dm * 32 + lrow];
#pragma unroll
                        for (int qt = 0; qt < QT; ++qt)
                            o[qt][dm] = mfma32x32x2f32(vf, s[k2][qt][v], o[qt][dm]);
                    }
                }
        }
        if (HPW == 1 && kb + 1 < nkb) store_block((kb + 1) & 1);
        __syncthreads();
    }

    if (!wave_active) return;
    float* ob = reinterpret_cast<float*>(p.out);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + qt * 32 + lrow;
        const float l_tot = l_run[qt] + __shfl_xor(l_run[qt], 32, 64);
        if (qi >= p.n_q) continue;
        const int64_t tok = tok_q(p, seq, qi);
        float scale = 1.0f / l_tot;
        if (p.gates) scale *= p.gates[tok * p.H + h];
        float* orow = ob + tok * p.ld_out + h * p.head_out;
#pragma unroll
        for (int dm = 0; dm < 2; ++dm)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d = dm * 32 + 8 * g + 4 * lh;
                f4 val;
#pragma unroll
                for (int e = 0; e < 4; ++e) val[e] = o[qt][dm][4 * g + e] * scale;
                *reinterpret_cast<f4*>(orow + d) = val;
            }
    }
}

// The DMA kernel addresses one (sequence, head) through a buffer descriptor
// based at its first key: every key row must lie within 2^31 bytes of it,
// and rows must be 16-byte aligned.
bool dma_fits(const AttnParams& p) {
    const int64_t rsb = p.k_pos * p.ld_in * 2;
    if (p.k_pos < 0 || p.ld_in % 8 != 0 || p.head_in % 8 != 0) return false;
    return (int64_t)(p.n_k - 1) * rsb + kD * 2 < ((int64_t)1 << 31);
}

int launch_attention(AttnParams& p, int64_t n_seq, int dtype, hipStream_t s) {
    const int hpw = p.n_q <= 64 && p.n_k <= 64 ? 4 : 1;
    const int wph = 4 / hpw;
    // Queries per wave: 64, or 32 for the fp32 one-head kernel (QT = 1: half
    // the Q / O / S registers, so two workgroups share a CU).
    const int qw = dtype == MSST_F32 && hpw == 1 ? 32 : 64;
    p.qtiles = (p.n_q + qw * wph - 1) / (qw * wph);
    const int64_t head_groups = (p.H + hpw - 1) / hpw;
    p.total_items = n_seq * head_groups * p.qtiles;
    // A q-tile covers qw * wph queries; the last one is reordered when at
    // least half of its waves are idle (with fewer, the q-tiles of a pair
    // running together in one L2 is worth more).
    p.short_last = p.qtiles * qw * wph - p.n_q >= qw / 2 * wph ? 1 : 0;
    // Grid: 8 XCDs x work items per XCD (whole pairs per XCD when the last
    // q-tiles are reordered, see work_item).
    const int64_t per_xcd = p.short_last ? (n_seq * head_groups + 7) / 8 * p.qtiles
                                         : (p.total_items + 7) / 8;
    if (per_xcd > 0x7fffffff / 8) return set_error(MSST_ERR_UNSUPPORTED, "attention grid too large");
    p.per_xcd = (int)per_xcd;
    const int64_t grid = per_xcd * 8;
    if (dtype == MSST_F16 && p.cos_t == nullptr && dma_fits(p)) {
        if (hpw == 4)
            hipLaunchKernelGGL(attn_f16_dma_kernel<4>, dim3((unsigned)grid), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(attn_f16_dma_kernel<1>, dim3((unsigned)grid), dim3(256), 0, s, p);
        return check_launch("attn_f16_dma_kernel");
    }
    if (dtype == MSST_F16) {
        if (hpw == 4)
            hipLaunchKernelGGL(attn_f16_kernel<4>, dim3((unsigned)grid), dim3(256), 0, s, p);
        else
            hipLaunchKernelGGL(attn_f16_kernel<1>, dim3((unsigned)grid), dim3(256), 0, s, p);
        return check_launch("attn_f16_kernel");
    }
    if (hpw == 4) {
        const size_t lds = 4 * 2 * kKB * kD * sizeof(float);
        hipLaunchKernelGGL((attn_f32_kernel<4, 2>), dim3((unsigned)grid), dim3(256), lds, s, p);
    } else {
        const size_t lds = 2 * 2 * kKB * kD * sizeof(float);
        hipLaunchKernelGGL((attn_f32_kernel<1, 1>), dim3((unsigned)grid), dim3(256), lds, s, p);
    }
    return check_launch("attn_f32_kernel");
}

// ===========================================================================
// Any head dim (msst_attention with D != 64)
// ===========================================================================
// The reference's scaled_dot_product_attention takes any head dim
// (ops_attention.cu:522-599: scores materialized through cuBLAS, softmax,
// then P.V).  D = 64, the Roformer head, runs the MFMA kernels above; any
// other D up to 256 runs this kernel: fp32 arithmetic for both dtypes and
// flash-style (online softmax over 32-key blocks staged in LDS as fp32), so
// nothing of size N x Nk is allocated.  A workgroup takes 64 queries of
// one (batch, head); thread (query ql, lane j < 4) holds dims j, j + 4, ...
// of its query's Q (pre-scaled by scale log2 e) and of O.  The four lanes
// of a query add their partial scores with two DPP quad permutes and then
// run the same online softmax.  LDS rows are DP = 4 NC floats, zero-filled
// past D, so the dot products need no per-dim predicate.
constexpr int kGenKB = 32;

__device__ __forceinline__ float quad_xor_sum(float x) {
    // quad_perm [1,0,3,2] (lane ^ 1), then [2,3,0,1] (lane ^ 2).
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, true));
    x += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x4E, 0xF, 0xF, true));
    return x;
}

template <typename T, int NC>
__global__ __launch_bounds__(256) void attn_generic_kernel(const T* __restrict__ q,
                                                           const T* __restrict__ k,
                                                           const T* __restrict__ v,
                                                           T* __restrict__ out, int N, int Nk,
                                                           int D, int qtiles, float scale_log2) {
    constexpr int DP = 4 * NC;
    __shared__ float Ks[kGenKB * DP], Vs[kGenKB * DP];
    const int64_t bh = blockIdx.x / qtiles;
    const int qt = (int)(blockIdx.x % qtiles);
    const int tid = threadIdx.x, ql = tid >> 2, j = tid & 3;
    const int qi = qt * 64 + ql;
    const bool qok = qi < N;
    const T* qrow = q + (bh * N + (qok ? qi : 0)) * D;
    float qv[NC], ov[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int d = j + 4 * c;
        qv[c] = (qok && d < D) ? (float)qrow[d] * scale_log2 : 0.0f;
        ov[c] = 0.0f;
    }
    const T* kbase = k + bh * Nk * D;
    const T* vbase = v + bh * Nk * D;
    float m = -INFINITY, l = 0.0f;
    for (int k0 = 0; k0 < Nk; k0 += kGenKB) {
        const int nk = min(kGenKB, Nk - k0);
        __syncthreads();  // every thread has finished reading the previous block
        for (int e = tid; e < kGenKB * DP; e += 256) {
            const int r = e / DP, d = e % DP;
            const bool ok = r < nk && d < D;
            const int64_t src = (int64_t)(k0 + r) * D + d;
            Ks[e] = ok ? (float)kbase[src] : 0.0f;
            Vs[e] = ok ? (float)vbase[src] : 0.0f;
        }
        __syncthreads();
        float sc[kGenKB];
        float bm = -INFINITY;
#pragma unroll
        for (int r = 0; r < kGenKB; ++r) {
            float acc = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) acc = fmaf(qv[c], Ks[r * DP + j + 4 * c], acc);
            acc = quad_xor_sum(acc);
            sc[r] = r < nk ? acc : -INFINITY;
            bm = fmaxf(bm, sc[r]);
        }
        const float m_new = fmaxf(m, bm);
        const float alpha = __builtin_amdgcn_exp2f(m - m_new);  // 0 for the first block
        l *= alpha;
#pragma unroll
        for (int c = 0; c < NC; ++c) ov[c] *= alpha;
#pragma unroll
        for (int r = 0; r < kGenKB; ++r) {
            const float pr = __builtin_amdgcn_exp2f(sc[r] - m_new);
            l += pr;
#pragma unroll
            for (int c = 0; c < NC; ++c) ov[c] = fmaf(pr, Vs[r * DP + j + 4 * c], ov[c]);
        }
        m = m_new;
    }
    if (!qok) return;
    T* orow = out + (bh * N + qi) * D;
    const float inv = 1.0f / l;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int d = j + 4 * c;
        if (d < D) orow[d] = (T)(ov[c] * inv);
    }
}

template <typename T, int NC>
int launch_generic_nc(const void* q, const void* k, const void* v, void* out, int64_t BH, int N,
                      int Nk, int D, int qtiles, float scale_log2, hipStream_t s) {
    hipLaunchKernelGGL((attn_generic_kernel<T, NC>), dim3((unsigned)(BH * qtiles)), dim3(256), 0,
                       s, static_cast<const T*>(q), static_cast<const T*>(k),
                       static_cast<const T*>(v), static_cast<T*>(out), N, Nk, D, qtiles,
                       scale_log2);
    return check_launch("attn_generic_kernel");
}

template <typename T>
int launch_generic(const void* q, const void* k, const void* v, void* out, int64_t BH, int N,
                   int Nk, int D, int qtiles, float scale_log2, hipStream_t s) {
    if (D <= 8) return launch_generic_nc<T, 2>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
    if (D <= 16) return launch_generic_nc<T, 4>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
    if (D <= 32) return launch_generic_nc<T, 8>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
    if (D <= 64) return launch_generic_nc<T, 16>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
    if (D <= 128)
        return launch_generic_nc<T, 32>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
    return launch_generic_nc<T, 64>(q, k, v, out, BH, N, Nk, D, qtiles, scale_log2, s);
}

bool fp32_lds_configured = false;

int configure_f32_lds() {
    if (fp32_lds_configured) return MSST_OK;
    // 128 KB of dynamic LDS for the 4-head fp32 variant (gfx950 has 160 KB).
    hipError_t e1 = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_f32_kernel<4, 2>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        4 * 2 * kKB * kD * (int)sizeof(float));
    hipError_t e2 = hipFuncSetAttribute(reinterpret_cast<const void*>(attn_f32_kernel<1, 1>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        2 * 2 * kKB * kD * (int)sizeof(float));
    if (e1 != hipSuccess || e2 != hipSuccess)
        return set_error(MSST_ERR_LAUNCH, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
    fp32_lds_configured = true;
    return MSST_OK;
}

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxGenericD = 4 * 64;

}  // namespace
}  // namespace msst

extern "C" int msst_attention(const void* q, const void* k, const void* v, void* out, int dtype,
                              int64_t B, int64_t H, int64_t N, int64_t Nk, int64_t D, float scale,
                              void* stream) {
    using namespace msst;
    MSST_REQUIRE(q && k && v && out, MSST_ERR_INVALID_ARG, "null tensor pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(B >= 0 && H >= 0 && N >= 0 && Nk >= 0, MSST_ERR_INVALID_ARG, "bad shape");
    MSST_REQUIRE(D >= 1 && D <= kMaxGenericD, MSST_ERR_UNSUPPORTED, "head dim must be in [1, 256]");
    MSST_REQUIRE(N < (1 << 30) && Nk < (1 << 30), MSST_ERR_UNSUPPORTED, "sequence too long");
    const size_t align = D == kD ? 16 : dtype_bytes(dtype);
    MSST_REQUIRE(aligned(q, align) && aligned(k, align) && aligned(v, align) && aligned(out, align),
                 MSST_ERR_ALIGNMENT,
                 D == kD ? "q, k, v, out must be 16-byte aligned"
                         : "q, k, v, out must be aligned to their element size");
    if (B * H == 0 || N == 0) return MSST_OK;
    MSST_REQUIRE(Nk > 0, MSST_ERR_INVALID_ARG, "no keys");
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)D);
    if (D != kD) {
        const int64_t qtiles = (N + 63) / 64;
        MSST_REQUIRE(B * H <= 0x7fffffff / qtiles, MSST_ERR_UNSUPPORTED, "attention grid too large");
        if (dtype == MSST_F32)
            return launch_generic<float>(q, k, v, out, B * H, (int)N, (int)Nk, (int)D, (int)qtiles,
                                         scale * kLog2e, as_stream(stream));
        return launch_generic<half_t>(q, k, v, out, B * H, (int)N, (int)Nk, (int)D, (int)qtiles,
                                      scale * kLog2e, as_stream(stream));
    }
    if (dtype == MSST_F32) {
        int rc = configure_f32_lds();
        if (rc) return rc;
    }
    AttnParams p{};
    p.q = q; p.k = k; p.v = v; p.out = out;
    p.ld_in = D; p.ld_out = D;
    p.cos_t = nullptr; p.sin_t = nullptr; p.gates = nullptr;
    p.n_inner = 1;
    p.n_q = (int)N; p.n_k = (int)Nk;
    p.scale_log2 = scale * kLog2e;
    // [B, H, N, D] as B sequences of H heads (head h of batch b at element
    // (b H + h) N D), so short sequences take the four-heads-per-workgroup
    // form; q and k/v share one head stride, so N != Nk runs B * H
    // one-head sequences instead.
    const bool heads = N == Nk && H <= (1 << 30);
    p.H = heads ? (int)H : 1;
    p.head_in = p.head_out = heads ? N * D : 0;
    p.q_outer = heads ? H * N : N; p.q_inner = 0; p.q_pos = 1;
    p.k_outer = heads ? H * Nk : Nk; p.k_inner = 0; p.k_pos = 1;
    return launch_attention(p, heads ? B : B * H, dtype, as_stream(stream));
}

extern "C" int msst_gated_rope_attention(const void* qkv, int dtype, int64_t ld_qkv,
                                         const float* cos_t, const float* sin_t,
                                         const float* gates, void* out, int64_t ld_out,
                                         const msst_seq_layout* layout, int H, int D, float scale,
                                         void* stream) {
    using namespace msst;
    MSST_REQUIRE(qkv && out && layout, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(is_dtype(dtype), MSST_ERR_INVALID_ARG, "bad dtype");
    MSST_REQUIRE(D == kD, MSST_ERR_UNSUPPORTED, "head dim must be 64");
    MSST_REQUIRE(H > 0 && ld_qkv >= 3LL * H * D && ld_out >= (int64_t)H * D,
                 MSST_ERR_INVALID_ARG, "row strides too small for 3*H*D / H*D");
    MSST_REQUIRE((cos_t == nullptr) == (sin_t == nullptr), MSST_ERR_INVALID_ARG,
                 "cos and sin tables must both be given or both be null");
    const msst_seq_layout& L = *layout;
    MSST_REQUIRE(L.n_outer >= 0 && L.n_inner >= 1 && L.seq_len >= 0 && L.seq_len < (1 << 30),
                 MSST_ERR_INVALID_ARG, "bad sequence layout");
    const size_t eb = dtype_bytes(dtype);
    MSST_REQUIRE(aligned(qkv, 16) && aligned(out, 16) && (ld_qkv * eb) % 16 == 0 &&
                     (ld_out * eb) % 16 == 0 && aligned(cos_t, 16) && aligned(sin_t, 16) &&
                     aligned(gates, 4),
                 MSST_ERR_ALIGNMENT, "qkv/out rows and RoPE tables must be 16-byte aligned");
    const int64_t n_seq = L.n_outer * L.n_inner;
    if (n_seq == 0 || L.seq_len == 0) return MSST_OK;
    if (dtype == MSST_F32) {
        int rc = configure_f32_lds();
        if (rc) return rc;
    }
    if (scale == 0.0f) scale = 1.0f / sqrtf((float)D);
    AttnParams p{};
    const char* base = reinterpret_cast<const char*>(qkv);
    p.q = base;
    p.k = base + (size_t)H * D * eb;
    p.v = base + (size_t)2 * H * D * eb;
    p.out = out;
    p.ld_in = ld_qkv; p.ld_out = ld_out; p.head_in = D; p.head_out = D;
    p.cos_t = cos_t; p.sin_t = sin_t; p.gates = gates;
    p.n_inner = L.n_inner;
    p.q_outer = p.k_outer = L.tok_outer;
    p.q_inner = p.k_inner = L.tok_inner;
    p.q_pos = p.k_pos = L.tok_pos;
    p.n_q = p.n_k = (int)L.seq_len;
    p.H = H;
    p.scale_log2 = scale * kLog2e;
    return launch_attention(p, n_seq, dtype, as_stream(stream));
}
