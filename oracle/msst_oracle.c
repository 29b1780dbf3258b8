/*
 * msst_oracle.c — CPU fp32 restatement of the Roformer transformer hot path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + timed CPU baseline); the
 * product never links it.  See msst_oracle.h for the per-function reference
 * citations and the deliberate departures (true fp32 instead of TF32,
 * precise libm instead of fast-math intrinsics).
 *
 * Parallelism: OpenMP over independent rows / (batch, head) pairs.  The GEMM
 * packs W into 16-column panels and runs a 6x16 register micro-tile written
 * with GCC vector extensions (AVX2 + FMA at -march=x86-64-v3).
 */
#include "msst_oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

typedef float v8f __attribute__((vector_size(32), aligned(4)));

#define MR 6
#define NR 16

int orc_num_threads(void) { return omp_get_max_threads(); }
void orc_set_num_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}

/* ops_fused.cu:21-24 (exact-erf GELU), :30-32 (sigmoid), :26-28 (SiLU). */
static inline float act_apply(float v, int act) {
    switch (act) {
    case ORC_ACT_GELU:
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    case ORC_ACT_SIGMOID:
        return 1.0f / (1.0f + expf(-v));
    case ORC_ACT_SILU:
        return v / (1.0f + expf(-v));
    case ORC_ACT_TANH:
        return tanhf(v);
    default:
        return v;
    }
}

void orc_activation(const float* x, float* out, int64_t n, int act) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = act_apply(x[i], act);
}

/* Pack W [N,K] (row-major) into panels of NR columns: panel p holds
 * Wp[p][k][c] = W[p*NR + c][k], zero beyond N. */
static float* pack_w(const float* w, int64_t K, int64_t N) {
    int64_t np = (N + NR - 1) / NR;
    float* wp = (float*)aligned_alloc(64, (size_t)(np * K * NR * sizeof(float) + 64));
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < np; ++p) {
        float* dst = wp + p * K * NR;
        for (int64_t k = 0; k < K; ++k)
            for (int c = 0; c < NR; ++c) {
                int64_t n = p * NR + c;
                dst[k * NR + c] = n < N ? w[n * K + k] : 0.0f;
            }
    }
    return wp;
}

/* Reference semantics: cuBLAS C = X.W^T (ops_linear.cu:176-185, :318-326),
 * then the bias kernel (ops_linear.cu:128-135) or the fused bias+activation
 * kernel (ops_fused.cu:40-102).  The optional residual is the caller's
 * `out + attn_out` (model_bs_roformer.cu:322, :326) folded in. */
void orc_linear(const float* x, const float* w, const float* b,
                const float* residual, float* out,
                int64_t M, int64_t K, int64_t N, int act) {
    if (M <= 0 || N <= 0) return;
    float* wp = pack_w(w, K, N);
    int64_t np = (N + NR - 1) / NR;
    int64_t mb = (M + MR - 1) / MR;
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t ib = 0; ib < mb; ++ib) {
        int64_t i0 = ib * MR;
        int rows = (int)((M - i0) < MR ? (M - i0) : MR);
        const float* arow[MR];
        for (int r = 0; r < MR; ++r) arow[r] = x + (i0 + (r < rows ? r : 0)) * K;
        for (int64_t p = 0; p < np; ++p) {
            const float* panel = wp + p * K * NR;
            v8f acc[MR][2];
            memset(acc, 0, sizeof(acc));
            for (int64_t k = 0; k < K; ++k) {
                v8f w0 = *(const v8f*)(panel + k * NR);
                v8f w1 = *(const v8f*)(panel + k * NR + 8);
                for (int r = 0; r < MR; ++r) {
                    float a = arow[r][k];
                    acc[r][0] += a * w0;
                    acc[r][1] += a * w1;
                }
            }
            for (int r = 0; r < rows; ++r) {
                int64_t i = i0 + r;
                for (int c = 0; c < NR; ++c) {
                    int64_t n = p * NR + c;
                    if (n >= N) break;
                    float v = acc[r][c >> 3][c & 7];
                    if (b) v += b[n];
                    v = act_apply(v, act);
                    if (residual) v += residual[i * N + n];
                    out[i * N + n] = v;
                }
            }
        }
    }
    free(wp);
}

/* ops_norm.cu:85-111: sum of squares over the row, rsqrt(ss + 1e-12),
 * times gamma and the caller's scale (sqrt(dim) at model_bs_roformer.cu:243). */
void orc_rms_norm(const float* x, const float* gamma, float scale, float* out,
                  int64_t rows, int64_t D) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* xi = x + r * D;
        float* yi = out + r * D;
        double ss = 0.0; /* summed in double: the oracle's ss has no
                            order-dependent rounding */
        for (int64_t j = 0; j < D; ++j) ss += (double)xi[j] * (double)xi[j];
        float inv = 1.0f / sqrtf((float)ss + 1e-12f);
        for (int64_t j = 0; j < D; ++j) yi[j] = xi[j] * inv * gamma[j] * scale;
    }
}

/* model_bs_roformer.cu:205-230 (identical in model_mel_band_roformer.cu:487-513). */
void orc_rope_table(int n, int dh, float* cos_out, float* sin_out) {
    int half = dh / 2;
    for (int p = 0; p < n; ++p)
        for (int i = 0; i < half; ++i) {
            float freq = 1.0f / powf(10000.0f, (float)(2 * i) / (float)dh);
            float angle = (float)p * freq;
            cos_out[p * half + i] = cosf(angle);
            sin_out[p * half + i] = sinf(angle);
        }
}

/* ops_misc.cu:39-69: pairs (2i, 2i+1) rotate by the angle of (n, i). */
void orc_rope_apply(float* q, float* k, const float* cos_t, const float* sin_t,
                    int64_t B, int64_t H, int64_t N, int64_t D) {
    int64_t half = D / 2;
#pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < B * H * N; ++row) {
        int64_t n = row % N;
        float* qr = q + row * D;
        float* kr = k + row * D;
        for (int64_t i = 0; i < half; ++i) {
            float c = cos_t[n * half + i], s = sin_t[n * half + i];
            float q0 = qr[2 * i], q1 = qr[2 * i + 1];
            qr[2 * i] = q0 * c - q1 * s;
            qr[2 * i + 1] = q0 * s + q1 * c;
            float k0 = kr[2 * i], k1 = kr[2 * i + 1];
            kr[2 * i] = k0 * c - k1 * s;
            kr[2 * i + 1] = k0 * s + k1 * c;
        }
    }
}

/* ops_attention.cu:96-181 (S = Q.K^T, softmax rows, O = P.V) and the
 * fused softmax of :390-452 (scale, row max, exp, sum, normalise). */
void orc_attention(const float* q, const float* k, const float* v, float* out,
                   int64_t B, int64_t H, int64_t N, int64_t Nk, int64_t D,
                   float scale) {
    int64_t BH = B * H;
#pragma omp parallel
    {
        float* srow = (float*)malloc((size_t)(Nk > 0 ? Nk : 1) * sizeof(float));
        float* acc = (float*)malloc((size_t)(D > 0 ? D : 1) * sizeof(float));
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int64_t bh = 0; bh < BH; ++bh) {
            for (int64_t i = 0; i < N; ++i) {
                const float* qi = q + (bh * N + i) * D;
                const float* kb = k + bh * Nk * D;
                const float* vb = v + bh * Nk * D;
                float mx = -INFINITY;
                int64_t D8 = D & ~(int64_t)7;
                for (int64_t j = 0; j < Nk; ++j) {
                    const float* kj = kb + j * D;
                    v8f s8 = {0, 0, 0, 0, 0, 0, 0, 0};
                    for (int64_t d = 0; d < D8; d += 8)
                        s8 += *(const v8f*)(qi + d) * *(const v8f*)(kj + d);
                    float s = ((s8[0] + s8[1]) + (s8[2] + s8[3])) +
                              ((s8[4] + s8[5]) + (s8[6] + s8[7]));
                    for (int64_t d = D8; d < D; ++d) s += qi[d] * kj[d];
                    s *= scale;
                    srow[j] = s;
                    if (s > mx) mx = s;
                }
                float sum = 0.0f;
                for (int64_t j = 0; j < Nk; ++j) {
                    float e = expf(srow[j] - mx);
                    srow[j] = e;
                    sum += e;
                }
                float inv = 1.0f / sum;
                for (int64_t d = 0; d < D; ++d) acc[d] = 0.0f;
                for (int64_t j = 0; j < Nk; ++j) {
                    float p = srow[j] * inv;
                    const float* vj = vb + j * D;
                    for (int64_t d = 0; d < D; ++d) acc[d] += p * vj[d];
                }
                float* oi = out + (bh * N + i) * D;
                for (int64_t d = 0; d < D; ++d) oi[d] = acc[d];
            }
        }
        free(srow);
        free(acc);
    }
}

/* model_mel_band_roformer.cu:34-52: qkv row layout is (qkv, h, d). */
void orc_split_qkv(const float* qkv, float* q, float* k, float* v,
                   int64_t B, int64_t N, int64_t H, int64_t D) {
    int64_t HD = H * D;
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n) {
            const float* row = qkv + (b * N + n) * 3 * HD;
            for (int64_t h = 0; h < H; ++h) {
                int64_t o = ((b * H + h) * N + n) * D;
                memcpy(q + o, row + h * D, (size_t)D * sizeof(float));
                memcpy(k + o, row + HD + h * D, (size_t)D * sizeof(float));
                memcpy(v + o, row + 2 * HD + h * D, (size_t)D * sizeof(float));
            }
        }
}

/* model_mel_band_roformer.cu:76-93 (BSR: model_bs_roformer.cu:266-278). */
void orc_gate_merge(const float* o, const float* gates, float* merged,
                    int64_t B, int64_t H, int64_t N, int64_t D) {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t n = 0; n < N; ++n)
            for (int64_t h = 0; h < H; ++h) {
                float g = gates[(b * N + n) * H + h];
                const float* src = o + ((b * H + h) * N + n) * D;
                float* dst = merged + (b * N + n) * H * D + h * D;
                for (int64_t d = 0; d < D; ++d) dst[d] = src[d] * g;
            }
}

static float* xalloc(int64_t n) {
    float* p = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!p) abort();
    return p;
}

/* model_bs_roformer.cu:236-331 / model_mel_band_roformer.cu:519-651. */
void orc_transformer(float* x, int64_t B, int64_t N, int64_t dim, int64_t H,
                     int64_t Dh, int64_t ff, const orc_layer_weights* w,
                     const float* cos_t, const float* sin_t) {
    int64_t M = B * N, HD = H * Dh;
    float scale = sqrtf((float)dim);
    float* normed = xalloc(M * dim);
    float* qkv = xalloc(M * 3 * HD);
    float* q = xalloc(M * HD);
    float* k = xalloc(M * HD);
    float* v = xalloc(M * HD);
    float* o = xalloc(M * HD);
    float* gates = xalloc(M * H);
    float* merged = xalloc(M * HD);
    float* hbuf = xalloc(M * ff);

    /* Attention block: model_bs_roformer.cu:242-283. */
    orc_rms_norm(x, w->attn_gamma, scale, normed, M, dim);
    orc_linear(normed, w->w_qkv, NULL, NULL, qkv, M, dim, 3 * HD, ORC_ACT_NONE);
    orc_split_qkv(qkv, q, k, v, B, N, H, Dh);
    orc_rope_apply(q, k, cos_t, sin_t, B, H, N, Dh);
    orc_attention(q, k, v, o, B, H, N, N, Dh, 1.0f / sqrtf((float)Dh));
    orc_linear(normed, w->w_gate, w->b_gate, NULL, gates, M, dim, H, ORC_ACT_SIGMOID);
    orc_gate_merge(o, gates, merged, B, H, N, Dh);
    /* x = x + to_out(merged)   (model_bs_roformer.cu:321-322) */
    orc_linear(merged, w->w_out, NULL, x, x, M, HD, dim, ORC_ACT_NONE);

    /* Feed-forward block: model_bs_roformer.cu:290-304, :325-326. */
    orc_rms_norm(x, w->ff_gamma, scale, normed, M, dim);
    orc_linear(normed, w->w_ff1, w->b_ff1, NULL, hbuf, M, dim, ff, ORC_ACT_GELU);
    orc_linear(hbuf, w->w_ff2, w->b_ff2, x, x, M, ff, dim, ORC_ACT_NONE);

    /* MelBandRoformer per-transformer output norm (:647-648). */
    if (w->final_gamma) {
        orc_rms_norm(x, w->final_gamma, scale, normed, M, dim);
        memcpy(x, normed, (size_t)(M * dim) * sizeof(float));
    }
    free(normed); free(qkv); free(q); free(k); free(v); free(o);
    free(gates); free(merged); free(hbuf);
}

/* [A,B',C',D'] <-> [A,C',B',D'] permute of the middle two axes. */
static void swap12(const float* src, float* dst, int64_t A, int64_t P, int64_t Q,
                   int64_t D) {
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t a = 0; a < A; ++a)
        for (int64_t p = 0; p < P; ++p)
            for (int64_t qq = 0; qq < Q; ++qq)
                memcpy(dst + ((a * Q + qq) * P + p) * D,
                       src + ((a * P + p) * Q + qq) * D, (size_t)D * sizeof(float));
}

/* model_bs_roformer.cu:482-539 / model_mel_band_roformer.cu:843-906. */
void orc_roformer_stack(float* x, int64_t B, int64_t T, int64_t F, int64_t dim,
                        int64_t H, int64_t Dh, int64_t ff, int64_t depth,
                        const orc_layer_weights* layers,
                        const float* final_gamma) {
    int64_t half = Dh / 2;
    float* tcos = xalloc(T * half);
    float* tsin = xalloc(T * half);
    float* fcos = xalloc(F * half);
    float* fsin = xalloc(F * half);
    orc_rope_table((int)T, (int)Dh, tcos, tsin);
    orc_rope_table((int)F, (int)Dh, fcos, fsin);
    float* tmp = xalloc(B * T * F * dim);
    for (int64_t d = 0; d < depth; ++d) {
        /* [B,T,F,dim] -> [B,F,T,dim]; time transformer on [B*F, T, dim]. */
        swap12(x, tmp, B, T, F, dim);
        orc_transformer(tmp, B * F, T, dim, H, Dh, ff, &layers[2 * d], tcos, tsin);
        /* back to [B,T,F,dim]; frequency transformer on [B*T, F, dim]. */
        swap12(tmp, x, B, F, T, dim);
        orc_transformer(x, B * T, F, dim, H, Dh, ff, &layers[2 * d + 1], fcos, fsin);
    }
    if (final_gamma) {
        orc_rms_norm(x, final_gamma, sqrtf((float)dim), tmp, B * T * F, dim);
        memcpy(x, tmp, (size_t)(B * T * F * dim) * sizeof(float));
    }
    free(tmp); free(tcos); free(tsin); free(fcos); free(fsin);
}

/* ops_elementwise.cu:321-344: first * 1 / (1 + exp(-second)). */
void orc_glu(const float* x, float* out, int64_t rows, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t j = 0; j < n; ++j) {
            const float a = x[r * 2 * n + j], g = x[r * 2 * n + n + j];
            out[r * n + j] = a * (1.0f / (1.0f + expf(-g)));
        }
}

/* model_bs_roformer.cu:337-368: split, per-band rms_norm with scale
 * sqrt(dims[b]), ops::linear, stack along dim 2. */
void orc_band_split(const float* x, int64_t rows, const int* dims, int nb,
                    const float* gamma, const float* w, const float* bias,
                    float* out, int64_t dim) {
    int64_t ftot = 0;
    for (int b = 0; b < nb; ++b) ftot += dims[b];
    int64_t off = 0;
    for (int b = 0; b < nb; ++b) {
        const int64_t d = dims[b];
        float* xb = (float*)malloc((size_t)(rows * d) * sizeof(float));
        float* ob = (float*)malloc((size_t)(rows * dim) * sizeof(float));
        for (int64_t r = 0; r < rows; ++r) memcpy(xb + r * d, x + r * ftot + off, (size_t)d * sizeof(float));
        orc_rms_norm(xb, gamma + off, sqrtf((float)d), xb, rows, d);
        orc_linear(xb, w + dim * off, bias + (int64_t)b * dim, NULL, ob, rows, d, dim, ORC_ACT_NONE);
        for (int64_t r = 0; r < rows; ++r)
            memcpy(out + (r * nb + b) * dim, ob + r * dim, (size_t)dim * sizeof(float));
        free(xb);
        free(ob);
        off += d;
    }
}

/* model_bs_roformer.cu:374-414: per band, linear -> tanh -> ... -> linear,
 * then glu(-1), concatenated along the last dimension. */
void orc_mask_estimator(const float* x, int64_t rows, const int* dims, int nb,
                        int64_t dim, int64_t hid, int L, const float* w,
                        const float* bias, float* out) {
    int64_t ftot = 0;
    for (int b = 0; b < nb; ++b) ftot += dims[b];
    int64_t off = 0, woff = 0, boff = 0;
    for (int b = 0; b < nb; ++b) {
        const int64_t d = dims[b];
        float* h = (float*)malloc((size_t)(rows * dim) * sizeof(float));
        for (int64_t r = 0; r < rows; ++r) memcpy(h + r * dim, x + (r * nb + b) * dim, (size_t)dim * sizeof(float));
        int64_t K = dim;
        for (int l = 0; l < L; ++l) {
            const int64_t N = (l == L - 1) ? 2 * d : hid;
            float* o = (float*)malloc((size_t)(rows * N) * sizeof(float));
            orc_linear(h, w + woff, bias + boff, NULL, o, rows, K, N,
                       l < L - 1 ? ORC_ACT_TANH : ORC_ACT_NONE);
            woff += N * K;
            boff += N;
            free(h);
            h = o;
            K = N;
        }
        float* g = (float*)malloc((size_t)(rows * d) * sizeof(float));
        orc_glu(h, g, rows, d);
        for (int64_t r = 0; r < rows; ++r) memcpy(out + r * ftot + off, g + r * d, (size_t)d * sizeof(float));
        free(g);
        free(h);
        off += d;
    }
}

/* model_bs_roformer.cu:450-469: permute [B,S,F,T,2] -> [B,F,S,T,2] (bins
 * interleave channels), index_select on the bin axis, permute to [B,T,bins,2]. */
void orc_band_gather(const float* stft, int64_t B, int64_t ch, int64_t F, int64_t T,
                     const int* fidx, int64_t n, float* out) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t)
            for (int64_t j = 0; j < n; ++j) {
                const int64_t g = fidx ? fidx[j] : j;
                const int64_t f = g / ch, s = g % ch;
                const float* src = stft + (((b * ch + s) * F + f) * T + t) * 2;
                out[((b * T + t) * n + j) * 2] = src[0];
                out[((b * T + t) * n + j) * 2 + 1] = src[1];
            }
}

/* model_mel_band_roformer.cu:924-1015: zeros, scatter_add (ops_misc.cu:395-440),
 * masks_summed / clamp(num_bands_per_freq, 1e-8), complex_mul
 * (ops_elementwise.cu:270-300), [B,N,F*S,T,2] -> [(B*N*S),F,T,2], index_fill. */
void orc_mask_merge(const float* masks, int64_t stems, const float* stft, int64_t B,
                    int64_t ch, int64_t F, int64_t T, const int* fidx, int64_t n,
                    int zero_dc, float* out) {
    const int64_t nbins = F * ch;
    float* cnt = (float*)calloc((size_t)nbins, sizeof(float));
    for (int64_t j = 0; j < n; ++j) cnt[fidx ? fidx[j] : j] += 1.0f;
    float* sum = (float*)malloc((size_t)(nbins * T * 2) * sizeof(float));
    for (int64_t nn = 0; nn < stems; ++nn)
        for (int64_t b = 0; b < B; ++b) {
            memset(sum, 0, (size_t)(nbins * T * 2) * sizeof(float));
            const float* mk = masks + ((nn * B + b) * T) * n * 2;
            for (int64_t t = 0; t < T; ++t)
                for (int64_t j = 0; j < n; ++j) {
                    const int64_t g = fidx ? fidx[j] : j;
                    sum[(g * T + t) * 2] += mk[(t * n + j) * 2];
                    sum[(g * T + t) * 2 + 1] += mk[(t * n + j) * 2 + 1];
                }
            for (int64_t g = 0; g < nbins; ++g) {
                const int64_t f = g / ch, s = g % ch;
                const float den = cnt[g] > 1e-8f ? cnt[g] : 1e-8f;
                for (int64_t t = 0; t < T; ++t) {
                    const float mr = sum[(g * T + t) * 2] / den, mi = sum[(g * T + t) * 2 + 1] / den;
                    const float* x = stft + (((b * ch + s) * F + f) * T + t) * 2;
                    float* o = out + ((((b * stems + nn) * ch + s) * F + f) * T + t) * 2;
                    o[0] = x[0] * mr - x[1] * mi;
                    o[1] = x[0] * mi + x[1] * mr;
                    if (zero_dc && f == 0) o[0] = o[1] = 0.0f;
                }
            }
        }
    free(sum);
    free(cnt);
}

/* In-place iterative radix-2 complex FFT in float64 (n a power of two);
 * sign -1 forward, +1 inverse (unnormalised). */
static void fft64(double* re, double* im, int n, int sign) {
    for (int i = 1, j = 0; i < n; ++i) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) {
            double t = re[i]; re[i] = re[j]; re[j] = t;
            t = im[i]; im[i] = im[j]; im[j] = t;
        }
    }
    for (int len = 2; len <= n; len <<= 1) {
        const double ang = sign * 2.0 * 3.14159265358979323846 / len;
        for (int i = 0; i < n; i += len)
            for (int k = 0; k < len / 2; ++k) {
                const double wr = cos(ang * k), wi = sin(ang * k);
                const int a = i + k, b = i + k + len / 2;
                const double xr = re[b] * wr - im[b] * wi, xi = re[b] * wi + im[b] * wr;
                re[b] = re[a] - xr; im[b] = im[a] - xi;
                re[a] += xr; im[a] += xi;
            }
    }
}

/* ops_stft.cu:286-362: pad_reflect, extract_frames_kernel, apply_window_kernel,
 * cufftExecR2C, complex_to_real_imag_kernel, stft_scale_kernel. */
void orc_stft(const float* signal, int64_t B, int64_t L, int n_fft, int hop,
              const float* window, int center, int normalized, float* out) {
    const int64_t pad = center ? n_fft / 2 : 0;
    const int64_t T = (L + 2 * pad - n_fft) / hop + 1;
    const int F = n_fft / 2 + 1;
    const double scale = normalized ? 1.0 / sqrt((double)n_fft) : 1.0;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t) {
            double* re = (double*)malloc(sizeof(double) * n_fft);
            double* im = (double*)malloc(sizeof(double) * n_fft);
            for (int n = 0; n < n_fft; ++n) {
                int64_t p = t * hop + n - pad;
                if (p < 0) p = -p;
                if (p >= L) p = 2 * (L - 1) - p;
                re[n] = (double)signal[b * L + p] * (double)window[n];
                im[n] = 0.0;
            }
            fft64(re, im, n_fft, -1);
            for (int k = 0; k < F; ++k) {
                float* o = out + ((b * F + k) * T + t) * 2;
                o[0] = (float)(re[k] * scale);
                o[1] = (float)(im[k] * scale);
            }
            free(re);
            free(im);
        }
}

/* ops_stft.cu:368-491: real_imag_to_complex, cufftExecC2R, / n_fft,
 * apply_window_kernel, overlap_add_kernel, window_sum_kernel,
 * normalize_by_window_kernel, centre slice, pad / slice to length. */
void orc_istft(const float* spec, int64_t B, int64_t T, int n_fft, int hop,
               const float* window, int64_t out_len, int center, int normalized, float* out) {
    const int F = n_fft / 2 + 1;
    const int64_t full = (int64_t)n_fft + (T - 1) * hop;
    const int64_t pad = center ? n_fft / 2 : 0;
    const double scale = normalized ? sqrt((double)n_fft) : 1.0;
    double* ola = (double*)calloc((size_t)(B * full), sizeof(double));
    double* wsum = (double*)calloc((size_t)full, sizeof(double));
    for (int64_t t = 0; t < T; ++t)
        for (int n = 0; n < n_fft; ++n) wsum[t * hop + n] += (double)window[n] * window[n];
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        double* re = (double*)malloc(sizeof(double) * n_fft);
        double* im = (double*)malloc(sizeof(double) * n_fft);
        for (int64_t t = 0; t < T; ++t) {
            for (int k = 0; k < F; ++k) {
                const float* s = spec + ((b * F + k) * T + t) * 2;
                re[k] = s[0] * scale;
                im[k] = (k == 0 || k == F - 1) ? 0.0 : s[1] * scale;
            }
            for (int k = F; k < n_fft; ++k) {  /* Hermitian extension */
                re[k] = re[n_fft - k];
                im[k] = -im[n_fft - k];
            }
            fft64(re, im, n_fft, +1);
            for (int n = 0; n < n_fft; ++n)
                ola[b * full + t * hop + n] += re[n] / n_fft * window[n];
        }
        free(re);
        free(im);
    }
    for (int64_t b = 0; b < B; ++b)
        for (int64_t o = 0; o < out_len; ++o) {
            const int64_t pos = o + pad;
            double v = 0.0;
            if (pos < full - pad) {
                v = ola[b * full + pos];
                if (wsum[pos] > 1e-8) v /= wsum[pos];
            }
            out[b * out_len + o] = (float)v;
        }
    free(ola);
    free(wsum);
}

/* ops_stft.cu:254-262 (periodic Hann, hann_window size 1 -> 1). */
void orc_hann_window(float* out, int size) {
    for (int i = 0; i < size; ++i)
        out[i] = size == 1 ? 1.0f
                           : (float)(0.5 * (1.0 - cos(2.0 * 3.14159265358979323846 * i / size)));
}

/* ops_misc.cu:469-525: mel = 2595 log10(1 + hz / 700); n_mels + 2 edges
 * evenly spaced in mel; bin f sits at sr * f / n_fft; rising edge on
 * [left, centre], falling edge on (centre, right]; all in float. */
void orc_mel_filterbank(float* out, int sr, int n_fft, int n_mels, float fmin, float fmax) {
    const int bins = n_fft / 2 + 1;
    if (fmax <= 0.0f) fmax = (float)sr / 2.0f;
    const float mlo = 2595.0f * log10f(1.0f + fmin / 700.0f);
    const float mhi = 2595.0f * log10f(1.0f + fmax / 700.0f);
    float* hz = (float*)malloc(sizeof(float) * (size_t)(n_mels + 2));
    for (int i = 0; i < n_mels + 2; ++i) {
        const float mel = mlo + (mhi - mlo) * (float)i / (float)(n_mels + 1);
        hz[i] = 700.0f * (powf(10.0f, mel / 2595.0f) - 1.0f);
    }
    for (int m = 0; m < n_mels; ++m) {
        const float l = hz[m], c = hz[m + 1], r = hz[m + 2];
        for (int f = 0; f < bins; ++f) {
            const float x = (float)sr * (float)f / (float)n_fft;
            float v = 0.0f;
            if (x >= l && x <= c) {
                if (c - l > 0.0f) v = (x - l) / (c - l);
            } else if (x > c && x <= r) {
                if (r - c > 0.0f) v = (r - x) / (r - c);
            }
            out[(size_t)m * bins + f] = v;
        }
    }
    free(hz);
}
