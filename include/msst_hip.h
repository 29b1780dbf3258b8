/*
 * msst_hip.h — C ABI of the MI355X (gfx950) Roformer hot path.
 *
 * This is the thin launcher layer beneath the C++ `cudasep::ops` / `Tensor`
 * API (cuda-msst-infer_amd/host/ops.h), which keeps the reference's
 * signatures.  Every entry point here:
 *   - takes raw device pointers, element counts and an explicit stream
 *     (`stream` is a hipStream_t; NULL means the null stream);
 *   - validates shapes, dtypes and alignment on the host BEFORE launching and
 *     returns MSST_OK (0) or a negative MSST_ERR_* code (message available
 *     through msst_last_error(), thread-local);
 *   - allocates nothing (the Roformer stack entry takes a caller workspace);
 *   - throws nothing.
 * Kernels are hand-written HIP for gfx950 (MFMA f16/f32, LDS-staged tiles);
 * no BLAS library is called.
 *
 * Reference interfaces replaced (CUDA-MSST-Infer, src/):
 *   msst_linear                 ops.h:65-66, :128-135  (ops_linear.cu:150-427,
 *                               ops_fused.cu:203-303, :341-358)
 *   msst_linear_rope            ops.h:66 + :99-100 fused (linear_no_bias of
 *                               to_qkv, then apply_rotary_emb on q and k,
 *                               model_bs_roformer.cu:249, :262)
 *   msst_band_split             model_bs_roformer.cu:337-368,
 *                               model_mel_band_roformer.cu:658-690 (per-band
 *                               rms_norm + linear + stack, one grouped launch)
 *   msst_mask_estimator         model_bs_roformer.cu:374-414,
 *                               model_mel_band_roformer.cu:696-738 (per-band
 *                               linear/tanh MLP + glu + cat, ops.h:36, :116)
 *   msst_band_gather            model_bs_roformer.cu:450-469,
 *                               model_mel_band_roformer.cu:792-820 (stereo merge,
 *                               index_select, permute into band features)
 *   msst_mask_merge             model_bs_roformer.cu:551-590,
 *                               model_mel_band_roformer.cu:924-1015 (stack,
 *                               scatter_add + mean, complex_mul ops.h:51,
 *                               stereo split, index_fill zero DC)
 *   msst_stft                   ops.h:87-89   (ops_stft.cu:286-362, cuFFT R2C)
 *   msst_istft                  ops.h:91-93   (ops_stft.cu:368-491, cuFFT C2R)
 *   msst_hann_window            ops.h:96      (ops_stft.cu:268-280)
 *   msst_chunk_extract          inference_app.cpp:116-156 (pad_reflect of the mix,
 *                               slice, pad_reflect / pad of the last chunk)
 *   msst_overlap_add            ops_fused.cu:138-168 (fused_overlap_add_kernel +
 *                               fused_weight_add_kernel)
 *   msst_normalize_by_weights   ops_fused.cu:170-186
 *   msst_band_plan_init         the per-band weight tables of
 *                               model_bs_roformer.h:65-70, :105-115
 *   msst_rms_norm               ops.h:56               (ops_norm.cu:455-491)
 *   msst_rms_norm_gate          ops.h:56 + :134 fused  (rms_norm followed by
 *                               linear_sigmoid, model_bs_roformer.cu:243, :268)
 *   msst_rope_table(_device)    model_bs_roformer.cu:205-230
 *   msst_rope_qk                ops.h:99-100           (ops_misc.cu:73-131)
 *   msst_attention              ops.h:83-85            (ops_attention.cu:522-599)
 *   msst_gated_rope_attention   model_bs_roformer.cu:250-278 (split heads,
 *                               RoPE, attention, gate, merge fused)
 *   msst_split_qkv_heads        model_mel_band_roformer.cu:34-74, :117-140
 *   msst_gate_merge_heads       model_mel_band_roformer.cu:76-115, :142-163
 *   msst_cast                   tensor.cu:1269-1294 (to_dtype)
 *   msst_add                    tensor.cu:1365-1447 (operator+, add_)
 *   msst_swap_axes12            tensor.cu:868-903 (permute + contiguous)
 *   msst_strided_copy           tensor.cu:868-903 (contiguous of a strided view),
 *                               :1062-1150 (cat, stack)
 *   msst_binary                 tensor.cu:1365-1447 (broadcast operator+ - * /,
 *                               add_, mul_)
 *   msst_tanh                   ops.h:36 tanh_act      (ops_elementwise.cu:84-88, :138)
 *   msst_complex_mul            ops.h:51 complex_mul   (ops_elementwise.cu:267-303)
 *   msst_glu                    ops.h:116 glu(x, -1)   (ops_elementwise.cu:321-388)
 *   msst_roformer_stack         model_bs_roformer.cu:482-539,
 *                               model_mel_band_roformer.cu:843-906
 *   msst_roformer_stack_layer   model_bs_roformer.cu:310-331 in the stack's
 *                               layout (transformer depth > 1, skip sums :477-487)
 *   msst_roformer_transformer   model_bs_roformer.cu:310-331,
 *                               model_mel_band_roformer.cu:621-651
 */
#ifndef MSST_HIP_H
#define MSST_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define MSST_OK 0
#define MSST_ERR_INVALID_ARG (-1)   /* null pointer, bad shape or dtype   */
#define MSST_ERR_UNSUPPORTED (-2)   /* shape/dtype combination not built  */
#define MSST_ERR_ALIGNMENT (-3)     /* pointer not aligned as required    */
#define MSST_ERR_LAUNCH (-4)        /* hipLaunch / runtime error          */
#define MSST_ERR_WORKSPACE (-5)     /* workspace too small                */

/* Element types: same values as cudasep::DType (tensor.h:15). */
#define MSST_F32 0
#define MSST_F16 1

/* Epilogue activations (ops_fused.cu:21-32). */
#define MSST_ACT_NONE 0
#define MSST_ACT_GELU 1    /* erf GELU, v Phi(v) (not the tanh form) */
#define MSST_ACT_SIGMOID 2
#define MSST_ACT_SILU 3

int msst_abi_version(void);
const char* msst_status_string(int status);
const char* msst_last_error(void);

/* out[M,N] = act(x[M,K] . W[N,K]^T + bias[N]) (+ residual[M,N]).
 * W is nn.Linear layout [out,in], row-major.  The compute precision follows
 * W's dtype as in the reference (ops_linear.cu:154): f16 W -> fp16 MFMA with
 * fp32 accumulation, f32 W -> fp32 MFMA.  x may be f32 or f16 (converted to
 * W's dtype as it is loaded).  bias (fp32) and residual (out_dtype) may be
 * NULL; residual may alias out.  out_dtype is f32 or f16. */
int msst_linear(const void* x, int x_dtype, const void* w, int w_dtype,
                const float* bias, const void* residual, void* out, int out_dtype,
                int64_t M, int64_t K, int64_t N, int act, void* stream);

/* fp16 out[M,N] = x[M,K] . w[N,K]^T (+ bias) with the interleaved-pair
 * rotary embedding applied to columns [0, rope_cols): the value is rounded
 * to fp16, then pair (2i, 2i+1) of each dim_head-wide head is rotated by
 * (cos_t, sin_t)[pos, i] in fp32 and rounded again, pos = (row / pos_div) %
 * pos_mod; tables are [pos_mod, dim_head / 2] fp32.  For a qkv projection
 * rope_cols = 2 * H * dim_head (q and k heads; v passes through).  x, w, out
 * f16.  Needs K % 64 == 0, rope_cols % 64 == 0, M < 2^24; otherwise
 * MSST_ERR_UNSUPPORTED (use msst_linear + msst_gated_rope_attention with
 * tables instead). */
int msst_linear_rope(const void* x, const void* w, const float* bias, void* out,
                     int64_t M, int64_t K, int64_t N, const float* cos_t,
                     const float* sin_t, int64_t rope_cols, int64_t dim_head,
                     int64_t pos_div, int64_t pos_mod, void* stream);

/* y = x * rsqrt(sum(x^2) + 1e-12) * gamma * scale per row of D elements. */
int msst_rms_norm(const void* x, int x_dtype, const float* gamma, float scale,
                  void* out, int out_dtype, int64_t rows, int64_t D,
                  void* stream);

/* msst_rms_norm, and in the same pass the attention gates
 * gates[r, g] = sigmoid(sum_d y_r[d] * w_gate[g, d] + b_gate[g]) for
 * g < G (G <= 16), computed from y rounded to out_dtype (what the
 * reference's linear_sigmoid would read).  w_gate [G, D] is f32 or f16. */
int msst_rms_norm_gate(const void* x, int x_dtype, const float* gamma,
                       float scale, void* out, int out_dtype,
                       const void* w_gate, int w_dtype, const float* b_gate,
                       float* gates, int64_t rows, int64_t D, int G,
                       void* stream);

/* Host-side RoPE table, [n, dim_head/2] each (model_bs_roformer.cu:205-230). */
int msst_rope_table(int n, int dim_head, float* cos_out, float* sin_out);

/* The same table computed on the device into device buffers (same float
 * formula; the device cosf/sinf may differ from the host's by an ulp). */
int msst_rope_table_device(int n, int dim_head, float* cos_out, float* sin_out,
                           void* stream);

/* In-place interleaved RoPE on q, k [B,H,N,D] (dtype f32 or f16); cos/sin
 * are fp32 device tables [N, D/2]. */
int msst_rope_qk(void* q, void* k, int dtype, const float* cos_t,
                 const float* sin_t, int64_t B, int64_t H, int64_t N, int64_t D,
                 void* stream);

/* out = softmax(scale * q.k^T) . v on contiguous [B,H,N,D] tensors
 * (k, v: [B,H,Nk,D]); dtype f32 (fp32 MFMA) or f16 (fp16 MFMA, fp32
 * softmax/accumulation).  scale == 0 means 1/sqrt(D).  D = 64 (the
 * Roformer head) runs the MFMA kernels and needs 16-byte aligned
 * pointers; any other D in [1, 256] runs an fp32 flash kernel (no N x Nk
 * buffer) and needs element-aligned pointers; D > 256 returns
 * MSST_ERR_UNSUPPORTED. */
int msst_attention(const void* q, const void* k, const void* v, void* out,
                   int dtype, int64_t B, int64_t H, int64_t N, int64_t Nk,
                   int64_t D, float scale, void* stream);

/* Token addressing of a batch of sequences inside a token-major buffer.
 * Sequence s = so * n_inner + si (so < n_outer, si < n_inner); position p of
 * it is token  so * tok_outer + si * tok_inner + p * tok_pos.
 *   time axis over [B,F,T] tokens:  n_outer=B*F n_inner=1 len=T
 *                                    tok_outer=T tok_inner=0 tok_pos=1
 *   freq axis over [B,F,T] tokens:  n_outer=B n_inner=T len=F
 *                                    tok_outer=F*T tok_inner=1 tok_pos=T */
typedef struct {
    int64_t n_outer, n_inner, seq_len;
    int64_t tok_outer, tok_inner, tok_pos;
} msst_seq_layout;

/* The Roformer attention block after the QKV projection, fused:
 * qkv rows [tokens, 3*H*D] (layout (qkv,h,d), row stride ld_qkv elements) ->
 * RoPE(q,k) over the sequence positions -> softmax(scale q.k^T) v ->
 * times gates[token*H + h] (NULL = 1) -> out[token, h*D + d] (row stride
 * ld_out).  cos/sin (NULL = no RoPE) are [seq_len, D/2] fp32.  dtype is the
 * element type of qkv and out.  D must be 64. */
int msst_gated_rope_attention(const void* qkv, int dtype, int64_t ld_qkv,
                              const float* cos_t, const float* sin_t,
                              const float* gates, void* out, int64_t ld_out,
                              const msst_seq_layout* layout, int H, int D,
                              float scale, void* stream);

/* [B,N,(3,H,D)] -> q,k,v [B,H,N,D] (same dtype). */
int msst_split_qkv_heads(const void* qkv, void* q, void* k, void* v, int dtype,
                         int64_t B, int64_t N, int64_t H, int64_t D,
                         void* stream);

/* merged[b,n,h*D+d] = attn[b,h,n,d] * gates[b,n,h]  (gates fp32). */
int msst_gate_merge_heads(const void* attn, const float* gates, void* merged,
                          int dtype, int64_t B, int64_t H, int64_t N, int64_t D,
                          void* stream);

/* Elementwise dtype conversion of n elements. */
int msst_cast(const void* src, int src_dtype, void* dst, int dst_dtype,
              int64_t n, void* stream);

/* out[i] = a[i] + b[i] (all of one dtype; out may alias a or b). */
int msst_add(const void* a, const void* b, void* out, int dtype, int64_t n,
             void* stream);

/* out[i] = a[i] * b[i] for n interleaved fp32 complex pairs (re, im); out
 * may alias a or b. */
int msst_complex_mul(const float* a, const float* b, float* out, int64_t n, void* stream);

/* out = tanh(x), elementwise (in place allowed). */
int msst_tanh(const void* x, void* out, int dtype, int64_t n, void* stream);

/* GLU over the last axis: out[r, j] = x[r, j] * sigmoid(x[r, j + half]),
 * x [rows, 2 * half], out [rows, half] (not aliased). */
int msst_glu(const void* x, void* out, int dtype, int64_t rows, int64_t half, void* stream);

/* dst[A,Q,P,R] = src[A,P,Q,R]: the permute({0,2,1,3}).contiguous() of the
 * depth loop (model_bs_roformer.cu:491, :509).  src and dst must differ. */
int msst_swap_axes12(const void* src, void* dst, int dtype, int64_t A,
                     int64_t P, int64_t Q, int64_t R, void* stream);

/* Strided views of cudasep::Tensor made real (tensor.cu:868-903 contiguous,
 * :1062-1150 cat / stack): dst[i] = src[i] for every index i of `shape`
 * (ndim <= 8), each side addressed by its own element strides (non-negative;
 * src strides may be 0 for broadcast axes, dst strides must not map two
 * indices to one element).  elem_bytes 1, 2, 4 or 8. */
int msst_strided_copy(const void* src, const int64_t* src_strides, void* dst,
                      const int64_t* dst_strides, const int64_t* shape, int ndim,
                      int elem_bytes, void* stream);

/* out = a op b elementwise over `shape` (ndim <= 8), out contiguous, a and b
 * addressed by element strides (0 along broadcast axes): Tensor operator+ -
 * * / and add_ / mul_ with broadcasting (tensor.cu:1365-1447).  fp16 is
 * computed in fp32 and rounded.  out may alias an operand that is
 * contiguous over `shape`. */
#define MSST_BIN_ADD 0
#define MSST_BIN_SUB 1
#define MSST_BIN_MUL 2
#define MSST_BIN_DIV 3
int msst_binary(const void* a, const int64_t* a_strides, const void* b,
                const int64_t* b_strides, void* out, const int64_t* shape, int ndim,
                int op, int dtype, void* stream);

/* Weights of one transformer (attention + feed-forward), as the Roformer
 * models hold them (model_bs_roformer.h:78-98).  Matrices are [out,in] in
 * the stack's weight dtype; gammas and biases are fp32.  final_gamma is the
 * MelBandRoformer per-transformer output norm (NULL for BSRoformer). */
typedef struct {
    const float* attn_gamma; /* [dim]         */
    const void* w_qkv;       /* [3*H*Dh, dim] */
    const void* w_gate;      /* [H, dim]      */
    const float* b_gate;     /* [H]           */
    const void* w_out;       /* [dim, H*Dh]   */
    const float* ff_gamma;   /* [dim]         */
    const void* w_ff1;       /* [ff, dim]     */
    const float* b_ff1;      /* [ff]          */
    const void* w_ff2;       /* [dim, ff]     */
    const float* b_ff2;      /* [dim]         */
    const float* final_gamma;/* [dim] or NULL */
} msst_layer_weights;

typedef struct {
    int64_t batch, frames, bands, dim, heads, dim_head, ff_dim, depth;
    int w_dtype; /* MSST_F16: fp16 weights/activations, fp32 residual and
                    accumulation; MSST_F32: fp32 throughout */
} msst_stack_desc;

/* Bytes of device workspace msst_roformer_stack needs for `desc`. */
int64_t msst_roformer_stack_workspace(const msst_stack_desc* desc);

/* The axial Roformer transformer stack, in place on the fp32 activation
 * x [batch, frames, bands, dim] (the layout the reference's depth loop
 * receives after band split).  layers holds 2*depth entries: time0, freq0,
 * time1, freq1, ...  final_gamma (BSRoformer's final norm) may be NULL.
 * workspace must hold msst_roformer_stack_workspace(desc) bytes, 256-byte
 * aligned.  No allocation, no host synchronisation. */
int msst_roformer_stack(float* x, const msst_stack_desc* desc,
                        const msst_layer_weights* layers,
                        const float* final_gamma, void* workspace,
                        int64_t workspace_bytes, void* stream);

/* One transformer (attention + feed-forward, and the MelBandRoformer
 * output norm when w->final_gamma is set) in place on the stack's fp32
 * activation x [batch, frames, bands, dim]: axis 0 attends over frames,
 * axis 1 over bands.  For the depth loops msst_roformer_stack does not
 * cover: time/freq_transformer_depth > 1 and skip connections
 * (model_bs_roformer.cu:310-331, :477-487, :531-535).  Same workspace as
 * msst_roformer_stack. */
int msst_roformer_stack_layer(float* x, const msst_stack_desc* desc,
                              const msst_layer_weights* w, int axis,
                              void* workspace, int64_t workspace_bytes,
                              void* stream);

/* msst_roformer_stack with no workspace argument and no allocation: the
 * workspace is the library's own static device scratch of
 * MSST_STACK_SCRATCH_BYTES per GPU.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops and harnesses that forbid hipMalloc).
 * Descriptors whose msst_roformer_stack_workspace(desc) exceeds the scratch
 * (about 10 800 tokens of a dim-512 stack) fail with MSST_ERR_WORKSPACE.
 * Every call on one GPU shares that GPU's scratch: calls that overlap on
 * one GPU (other streams, other host threads) race and must be serialised
 * by the caller.  Nothing in the scratch needs to start at zero. */
#define MSST_STACK_SCRATCH_BYTES (64LL << 20)
int msst_roformer_stack_noalloc(float* x, const msst_stack_desc* desc,
                                const msst_layer_weights* layers,
                                const float* final_gamma, void* stream);

/* One transformer (apply_transformer with depth 1, model_bs_roformer.cu:
 * 310-331 / model_mel_band_roformer.cu:621-651) in place on the fp32
 * activation x in time-major token order [batch, bands, frames, dim]:
 * axis 0 attends over frames (the time layer), axis 1 over bands.  Same
 * workspace as msst_roformer_stack (desc.depth is ignored). */
int msst_roformer_transformer(float* x, const msst_stack_desc* desc,
                              const msst_layer_weights* w, int axis,
                              void* workspace, int64_t workspace_bytes,
                              void* stream);

/* ---- Band split and mask estimator (grouped over bands) -----------------
 * Bands: band b owns band_dims[b] consecutive features (2 * frequencies *
 * audio channels) of the [rows, sum(band_dims)] STFT feature row.  The
 * per-band weights stay in the caller's tensors; msst_band_plan_init copies
 * their addresses into `plan` (device memory of msst_band_plan_bytes) once
 * per model and packs the band-split weights into zero-padded rows.  A plan
 * holds the band split and/or one stem's mask estimator (pass NULL for the
 * part it does not hold).  fp16 weights (W), fp32 gamma / bias. */
typedef struct msst_band_config {
    int num_bands;         /* 1..64                                           */
    const int* band_dims;  /* host array [num_bands]: even, 2..1024           */
    int dim;               /* model dim (multiple of 64)                      */
    int hidden;            /* mask-estimator hidden width (multiple of 64)    */
    int mlp_linears;       /* linears per band MLP (BSRoformer: mask_estimator_depth,
                              MelBandRoformer: mask_estimator_depth + 1); 1..8 */
    /* STFT side (msst_band_gather / msst_mask_merge only; 0 / NULL otherwise): */
    int audio_channels;    /* 1 or 2; bin g = f * audio_channels + s interleaves stereo */
    int stft_bins;         /* F = n_fft / 2 + 1                                */
    const int* freq_indices; /* host [sum(band_dims) / 2]: the interleaved bin of each band
                              feature pair (MelBandRoformer's freq_indices_,
                              model_mel_band_roformer.cu:238-268); NULL = bins in
                              order, every bin once (BSRoformer)               */
} msst_band_config;

int64_t msst_band_plan_bytes(const msst_band_config* c);

/* split_gamma[b] f32 [band_dims[b]], split_w[b] f16 [dim, band_dims[b]],
 * split_b[b] f32 [dim]; mask_w[b * L + l] f16 [N_l, K_l] (K_0 = dim, N_l =
 * hidden below the last layer, N_{L-1} = 2 band_dims[b]), mask_b likewise.
 * Pointer arrays are host arrays of device pointers.  Synchronous: returns
 * after the plan is written.  plan 256-byte aligned. */
int msst_band_plan_init(const msst_band_config* c, const float* const* split_gamma,
                        const void* const* split_w, const float* const* split_b,
                        const void* const* mask_w, const float* const* mask_b,
                        void* plan, int64_t plan_bytes, void* stream);

/* out[r, b, :] = rms_norm(x[r, band b], gamma_b, sqrt(band_dims[b])) . W_b^T
 * + bias_b.  x f32 [rows, sum(band_dims)], out f32 [rows, num_bands, dim]
 * (the reference's stack along dim 2).  The normalised bands are rounded to
 * fp16, as ops::linear casts its input.  Workspace: msst_band_split_workspace
 * bytes, 16-byte aligned. */
int64_t msst_band_split_workspace(const msst_band_config* c, int64_t rows);
int msst_band_split(const msst_band_config* c, const void* plan, const float* x,
                    int64_t rows, float* out, void* workspace, int64_t ws_bytes,
                    void* stream);

/* One stem's mask estimator: for every band b, the MLP (tanh between
 * linears) on x[:, b, :] followed by glu; out f32 [rows, sum(band_dims)]
 * with band b at its feature offset (the reference's cat).  x f32 or f16
 * [rows, num_bands, dim] (fp32 input is cast to fp16 as ops::linear does);
 * hidden activations are kept in fp16.  Workspace:
 * msst_mask_estimator_workspace bytes, 256-byte aligned. */
int64_t msst_mask_estimator_workspace(const msst_band_config* c, int64_t rows);
int msst_mask_estimator(const msst_band_config* c, const void* plan, const void* x,
                        int x_dtype, int64_t rows, float* out, void* workspace,
                        int64_t ws_bytes, void* stream);

/* STFT -> band-split input (model_bs_roformer.cu:450-469,
 * model_mel_band_roformer.cu:792-820: stereo merge into the bin axis, the
 * freq_indices gather, complex folded into features):
 *   out[b, t, 2 j + c] = stft[b * ch + s, f, t, c],  f * ch + s = freq_indices[j].
 * stft f32 [batch * ch, F, frames, 2] (the STFT's layout), out f32
 * [batch, frames, sum(band_dims)].  Needs the plan's STFT side. */
int msst_band_gather(const msst_band_config* c, const void* plan, const float* stft,
                     int64_t batch, int64_t frames, float* out, void* stream);

/* Masks -> masked STFT, ready for the iSTFT (model_bs_roformer.cu:551-590,
 * model_mel_band_roformer.cu:924-1015): each bin's mask is the mean over the
 * bands that hold it (scatter_add / num_bands_per_freq, clamped at 1e-8; a
 * plain copy for BSRoformer), complex-multiplied with the STFT, stereo
 * un-interleaved, bin 0 zeroed when zero_dc:
 *   out[(b * stems + n) * ch + s, f, t] = stft[b * ch + s, f, t] * mask_n[b, t, f * ch + s].
 * masks f32 [stems][batch, frames, sum(band_dims)] (each stem's
 * msst_mask_estimator output, stem-major), stft as above, out f32
 * [batch * stems * ch, F, frames, 2].  The sums run in a fixed order
 * (deterministic).  Workspace: msst_mask_merge_workspace bytes (0 for
 * in-order bins), 16-byte aligned. */
int64_t msst_mask_merge_workspace(const msst_band_config* c, int64_t batch, int64_t stems,
                                  int64_t frames);
int msst_mask_merge(const msst_band_config* c, const void* plan, const float* masks,
                    int64_t stems, const float* stft, int64_t batch, int64_t frames,
                    int zero_dc, float* out, void* workspace, int64_t ws_bytes, void* stream);

/* ---- Chunked inference (inference_app.cpp:100-324) --------------------------
 * dst [channels, chunk] = samples [start, start + chunk) of the audio
 * [channels, length] reflect-padded by `border` on both sides (border <
 * length); past its end, the chunk's own slice reflect-padded at its end
 * (tail_reflect; needs more than half a chunk of signal) or zero. */
int msst_chunk_extract(const float* audio, int64_t channels, int64_t length, int64_t border,
                       int64_t start, int64_t chunk, int tail_reflect, float* dst, void* stream);

/* out[c, offset + i] += src[c * src_stride + i] * window[i] and
 * wsum[offset + i] += window[i] for i < len; out [channels, total].  Calls
 * on one stream apply in order (no atomics: run to run identical). */
int msst_overlap_add(float* out, float* wsum, const float* src, int64_t src_stride,
                     const float* window, int64_t channels, int64_t total, int64_t offset,
                     int64_t len, void* stream);

/* out[c, i] /= wsum[i] where wsum[i] > 1e-8. */
int msst_normalize_by_weights(float* out, const float* wsum, int64_t channels, int64_t total,
                              void* stream);

/* ---- STFT / iSTFT (torch.stft / torch.istft semantics, as the reference) --
 * Hand-written FFT (power-of-two n_fft in [16, 4096]); the window has n_fft
 * samples (win_length == n_fft, as the reference's kernels index it).
 *
 * out[b, k, t] = sum_n x_b[t * hop + n - pad] w[n] exp(-2 pi i k n / n_fft),
 * k = 0..n_fft/2, pad = n_fft/2 with reflect padding when center (needs
 * length > n_fft/2), times 1/sqrt(n_fft) when normalized.  signal f32
 * [batch, length], out f32 [batch, n_fft/2 + 1, frames, 2] with frames =
 * msst_stft_frames(...). */
int64_t msst_stft_frames(int64_t length, int n_fft, int hop, int center);
int msst_stft(const float* signal, int64_t batch, int64_t length, int n_fft, int hop,
              const float* window, int center, int normalized, float* out, void* stream);

/* Inverse: per frame the Hermitian C2R transform (imaginary parts of bins 0
 * and n_fft/2 ignored) / n_fft, windowed, overlap-added in frame order and
 * divided by sum_t w^2 where that exceeds 1e-8; the centre padding is
 * trimmed and the result truncated or zero-padded to `length` (> 0), else
 * msst_istft_length(...) samples.  spec f32 [batch, n_fft/2 + 1, frames, 2],
 * out f32 [batch, out_len].  Workspace: msst_istft_workspace bytes. */
int64_t msst_istft_length(int64_t frames, int n_fft, int hop, int64_t length, int center);
int64_t msst_istft_workspace(int64_t batch, int64_t frames, int n_fft);
int msst_istft(const float* spec, int64_t batch, int64_t frames, int n_fft, int hop,
               const float* window, int64_t length, int center, int normalized, float* out,
               void* workspace, int64_t ws_bytes, void* stream);

/* Periodic Hann window, w[i] = (1 - cos(2 pi i / size)) / 2 (size 1: 1). */
int msst_hann_window(float* out, int size, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* MSST_HIP_H */
