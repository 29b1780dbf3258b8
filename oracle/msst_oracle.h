/*
 * msst_oracle.h — CPU fp32 restatement of the Roformer transformer hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * kernels and the timed CPU baseline of the benchmark.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product (libmsst_hip.so, libcudasep_amd.so) never links or calls it.
 *
 * Every function restates the arithmetic of the reference file:line it cites
 * (paths relative to the CUDA-MSST-Infer source tree).  Deliberate departures:
 *   - GEMMs are true fp32 (the reference runs cuBLAS in TF32 for fp32 and
 *     16F x 16F -> 32F for fp16 weights); the target of the port is fp32.
 *   - expf / erff are the precise libm routines (the reference is compiled
 *     with --use_fast_math and uses __expf in its softmax).
 * Layout conventions follow the reference: row-major, W is nn.Linear [out,in].
 */
#ifndef MSST_ORACLE_H
#define MSST_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_ACT_NONE = 0, ORC_ACT_GELU = 1, ORC_ACT_SIGMOID = 2, ORC_ACT_SILU = 3, ORC_ACT_TANH = 4 };

/* Weights of one transformer (attention + feed-forward) as the two Roformer
 * models hold them (model_bs_roformer.h:78-98). final_gamma is the
 * MelBandRoformer per-transformer output norm
 * (model_mel_band_roformer.cu:647-648); NULL for BSRoformer. */
typedef struct {
    const float* attn_gamma; /* [dim]              */
    const float* w_qkv;      /* [3*H*Dh, dim]      */
    const float* w_gate;     /* [H, dim]           */
    const float* b_gate;     /* [H]                */
    const float* w_out;      /* [dim, H*Dh]        */
    const float* ff_gamma;   /* [dim]              */
    const float* w_ff1;      /* [ff, dim]          */
    const float* b_ff1;      /* [ff]               */
    const float* w_ff2;      /* [dim, ff]          */
    const float* b_ff2;      /* [dim]              */
    const float* final_gamma;/* [dim] or NULL      */
} orc_layer_weights;

int orc_num_threads(void);
void orc_set_num_threads(int n);

/* out[M,N] = act(x[M,K] . W[N,K]^T + b) (+ residual). b / residual may be
 * NULL.  ops_linear.cu:150-193, :349-427; ops_fused.cu:203-303, :341-358. */
void orc_linear(const float* x, const float* w, const float* b,
                const float* residual, float* out,
                int64_t M, int64_t K, int64_t N, int act);

/* Elementwise activations (ops_fused.cu:21-32; tanh: ops_elementwise.cu:84-88). */
void orc_activation(const float* x, float* out, int64_t n, int act);

/* y = x * rsqrt(sum(x^2) + 1e-12) * gamma * scale per row
 * (ops_norm.cu:85-111, :455-491). */
void orc_rms_norm(const float* x, const float* gamma, float scale, float* out,
                  int64_t rows, int64_t D);

/* Host RoPE table: freq_i = 1/10000^(2i/dh), angle = n*freq_i, all in float
 * (model_bs_roformer.cu:205-230).  cos/sin: [n, dh/2]. */
void orc_rope_table(int n, int dh, float* cos_out, float* sin_out);

/* In-place interleaved-pair rotation of q and k [B,H,N,D]
 * (ops_misc.cu:39-69). */
void orc_rope_apply(float* q, float* k, const float* cos_t, const float* sin_t,
                    int64_t B, int64_t H, int64_t N, int64_t D);

/* out[B,H,N,D] = softmax(scale * q.k^T) . v   (ops_attention.cu:96-181,
 * :390-452, :522-599). */
void orc_attention(const float* q, const float* k, const float* v, float* out,
                   int64_t B, int64_t H, int64_t N, int64_t Nk, int64_t D,
                   float scale);

/* [B,N,(3,H,D)] -> 3 x [B,H,N,D]   (model_mel_band_roformer.cu:34-52). */
void orc_split_qkv(const float* qkv, float* q, float* k, float* v,
                   int64_t B, int64_t N, int64_t H, int64_t D);

/* merged[b,n,h*D+d] = o[b,h,n,d] * gates[b,n,h]
 * (model_mel_band_roformer.cu:76-93). */
void orc_gate_merge(const float* o, const float* gates, float* merged,
                    int64_t B, int64_t H, int64_t N, int64_t D);

/* One transformer on x [B,N,dim], in place: x += Attn(x); x += FF(x);
 * then the optional final norm (model_bs_roformer.cu:236-331,
 * model_mel_band_roformer.cu:519-651).  cos/sin: [N, Dh/2]. */
void orc_transformer(float* x, int64_t B, int64_t N, int64_t dim, int64_t H,
                     int64_t Dh, int64_t ff, const orc_layer_weights* w,
                     const float* cos_t, const float* sin_t);

/* Axial stack on x [B,T,F,dim], in place.  layers holds 2*depth entries in
 * the order time0, freq0, time1, freq1, ...; each depth permutes to
 * [B,F,T,dim], runs the time transformer on [B*F,T,dim], permutes back and
 * runs the frequency transformer on [B*T,F,dim] (model_bs_roformer.cu:482-534,
 * model_mel_band_roformer.cu:843-906).  final_gamma (BSRoformer,
 * model_bs_roformer.cu:538-539) may be NULL. */
void orc_roformer_stack(float* x, int64_t B, int64_t T, int64_t F, int64_t dim,
                        int64_t H, int64_t Dh, int64_t ff, int64_t depth,
                        const orc_layer_weights* layers,
                        const float* final_gamma);

/* GLU over the last dimension: out[r, j] = x[r, j] * sigmoid(x[r, j + n]) for
 * x [rows, 2n] (ops_elementwise.cu:321-388). */
void orc_glu(const float* x, float* out, int64_t rows, int64_t n);

/* Band split (model_bs_roformer.cu:337-368; model_mel_band_roformer.cu:658-690).
 * x [rows, sum(dims)]: band b is columns [off_b, off_b + dims[b]).  For each
 * band: y = rms_norm(x_b, gamma_b, sqrt(dims[b])), out[r, b, :] = y . W_b^T +
 * bias_b.  gamma: the gamma_b concatenated [sum(dims)]; w: the W_b [dim,
 * dims[b]] concatenated (band b at dim * off_b); bias [nb, dim];
 * out [rows, nb, dim]. */
void orc_band_split(const float* x, int64_t rows, const int* dims, int nb,
                    const float* gamma, const float* w, const float* bias,
                    float* out, int64_t dim);

/* Mask estimator of one stem (model_bs_roformer.cu:374-414;
 * model_mel_band_roformer.cu:696-738).  x [rows, nb, dim].  Per band b: an
 * MLP of L linears, tanh between them (not after the last), widths dim ->
 * hid -> ... -> hid -> 2 dims[b], then GLU; the result fills columns
 * [off_b, off_b + dims[b]) of out [rows, sum(dims)].  w / bias hold the
 * layers in (band, layer) order, each W [N_l, K_l] row-major. */
void orc_mask_estimator(const float* x, int64_t rows, const int* dims, int nb,
                        int64_t dim, int64_t hid, int L, const float* w,
                        const float* bias, float* out);

/* STFT -> band features (model_bs_roformer.cu:450-469,
 * model_mel_band_roformer.cu:792-820): stft [B*ch, F, T, 2]; the stereo
 * channels are merged into the bin axis (g = f*ch + s), bins are gathered by
 * fidx [n] (NULL: g = j) and complex is folded into the features:
 * out[b, t, 2j + c] = stft[b*ch + s, f, t, c].  out [B, T, 2n]. */
void orc_band_gather(const float* stft, int64_t B, int64_t ch, int64_t F, int64_t T,
                     const int* fidx, int64_t n, float* out);

/* Masks -> masked STFT (model_mel_band_roformer.cu:924-1015, and
 * model_bs_roformer.cu:551-590 with fidx NULL): scatter_add of each stem's
 * mask pairs into the bins, division by the number of bands per bin
 * (clamped at 1e-8), complex_mul with the STFT, stereo un-interleave and
 * index_fill of bin 0 when zero_dc.  masks [stems][B, T, 2n];
 * out [(B*stems*ch), F, T, 2]. */
void orc_mask_merge(const float* masks, int64_t stems, const float* stft, int64_t B,
                    int64_t ch, int64_t F, int64_t T, const int* fidx, int64_t n,
                    int zero_dc, float* out);

/* torch.stft semantics (ops_stft.cu:286-362): reflect-pad n_fft/2 each side
 * when center, frames at hop, window [n_fft], one-sided FFT (float64 radix-2
 * here), times 1/sqrt(n_fft) when normalized.  signal [B, L] ->
 * out [B, n_fft/2 + 1, T, 2], T = (L + (center ? n_fft : 0) - n_fft) / hop + 1. */
void orc_stft(const float* signal, int64_t B, int64_t L, int n_fft, int hop,
              const float* window, int center, int normalized, float* out);

/* torch.istft semantics (ops_stft.cu:368-491): C2R per frame / n_fft (imaginary
 * parts of bins 0 and n_fft/2 ignored), window, overlap-add, division by the
 * squared-window sum where > 1e-8, centre trim, truncate / zero-pad to
 * `length` (> 0).  spec [B, n_fft/2 + 1, T, 2] -> out [B, out_len]. */
void orc_istft(const float* spec, int64_t B, int64_t T, int n_fft, int hop,
               const float* window, int64_t out_len, int center, int normalized, float* out);

/* Periodic Hann window (ops_stft.cu:254-262). */
void orc_hann_window(float* out, int size);

/* Triangular HTK-mel filterbank out[n_mels, n_fft/2 + 1] in float, step for
 * step as ops_misc.cu:469-525 (fmax <= 0 -> sr / 2). */
void orc_mel_filterbank(float* out, int sr, int n_fft, int n_mels, float fmin, float fmax);

#ifdef __cplusplus
}
#endif
#endif
