// ops.h — the reference's `cudasep::ops` surface for the Roformer hot path
// (src/ops.h:10-28, :56, :65-66, :83-85, :99-100, :128-135), on MI355X.
//
// Each function keeps the reference's name, signature, argument meaning and
// dtype rules, and launches the hand-written gfx950 kernels through the C
// ABI (include/msst_hip.h).  Errors become std::runtime_error carrying the
// ABI's message (the reference throws the same type from CUDA_CHECK; its
// shape asserts are checks that throw here).
//
// Dtype rules (the reference's):
//   - a GEMM's precision is chosen by the WEIGHT dtype: fp16 W -> fp16 MFMA
//     with fp32 accumulation (x is rounded to fp16 as it is loaded); fp32 W
//     -> fp32 MFMA;
//   - linear / linear_no_bias with fp16 W return fp32 (ops_linear.cu:192,
//     :384); with fp32 W they return x's dtype;
//   - linear_gelu / linear_sigmoid / linear_silu return fp16 when x is fp16,
//     else fp32 (ops_fused.cu:280, :301);
//   - rms_norm, apply_rotary_emb and scaled_dot_product_attention keep the
//     input dtype; fp16 biases / gammas / tables are promoted to fp32.
// Numerics differ from the reference where it uses TF32 (its "fp32" GEMMs
// and QK^T): fp32 here is true fp32 MFMA.
//
// Streams: every op runs on CudaContext::instance().stream() (the null
// stream unless set_stream() chose another).  Not re-entrant across
// threads, like the reference.
#pragma once

#include <vector>

#include "msst_hip.h"
#include "tensor.h"

namespace cudasep {

// fp16 switch of the reference (ops_linear.cu:16): read by the weight loader
// to convert 2-D weights to fp16.  The ops here follow the weight dtype.
extern bool g_quantize_fp16;
// The reference captures its materialised attention into CUDA graphs
// (ops_attention.cu:183-380).  The fused flash kernel here has no
// per-shape state, so the flag is accepted and ignored, and clearing the
// cache is a no-op.
extern bool g_enable_cuda_graph_attention;
void clear_attention_graph_cache();

// Process-wide context (the reference's CudaContext, ops.h:14-28, minus the
// cuBLAS/cuDNN handles: no library is called on this path).
class CudaContext {
public:
    static CudaContext& instance();
    hipStream_t stream() { return stream_; }
    void set_stream(hipStream_t s) { stream_ = s; }
    void sync();  // hipDeviceSynchronize

private:
    CudaContext() = default;
    hipStream_t stream_ = nullptr;
};

namespace ops {

Tensor rms_norm(const Tensor& x, const Tensor& gamma, float scale);

Tensor linear(const Tensor& x, const Tensor& weight, const Tensor& bias);  // x @ W^T + b
Tensor linear_no_bias(const Tensor& x, const Tensor& weight);             // x @ W^T

// q,k,v: [B, H, N, D] (D = 64); scale 0 -> 1/sqrt(D); dropout ignored.
Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v,
                                    float scale = 0.0f, float dropout = 0.0f);

// q,k: [B, H, N, D] rotated in place (interleaved pairs); cos/sin [N, D/2].
void apply_rotary_emb(Tensor& q, Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs);

// ops.h:87-96 (ops_stft.cu): torch.stft / torch.istft semantics on a
// hand-written FFT (power-of-two n_fft in [16, 4096]; win_length must equal
// n_fft, as the reference's kernels index the window by n_fft).
// stft: signal [B, L] (or [L]) -> [B, n_fft/2 + 1, T, 2] fp32.
// istft: [B, F, T, 2] -> [B, length or the full trimmed length] fp32.
Tensor stft(const Tensor& signal, int n_fft, int hop_length, int win_length,
            const Tensor& window, bool center = true, bool normalized = false);
Tensor istft(const Tensor& complex_spec, int n_fft, int hop_length, int win_length,
             const Tensor& window, int64_t length = -1, bool center = true,
             bool normalized = false);
Tensor hann_window(int size);

// ops.h:124 (ops_misc.cu:469-525): triangular HTK-mel filterbank
// [n_mels, n_fft/2 + 1] (mel = 2595 log10(1 + f/700); n_mels + 2 points
// evenly spaced in mel between fmin and fmax, fmax <= 0 meaning sr / 2;
// bin f at sr * f / n_fft), computed in float on the host like the
// reference's.  mel_filterbank_host returns the row-major values,
// mel_filterbank the same uploaded to the device.
std::vector<float> mel_filterbank_host(int sr, int n_fft, int n_mels, float fmin = 0.0f,
                                       float fmax = 0.0f);
Tensor mel_filterbank(int sr, int n_fft, int n_mels, float fmin = 0.0f, float fmax = 0.0f);

// ops_elementwise.cu:84-88, :138 (tanhf) and :321-388 (first * sigmoid(second));
// glu splits the last dimension only (the Roformers' use, dim = -1).
Tensor tanh_act(const Tensor& x);
Tensor glu(const Tensor& x, int dim = -1);

// ops.h:51 and :121 (ops_elementwise.cu:267-303, :503-527): the mask side of
// the Roformers' forward (the masked STFT, the zeroed DC bin).
// complex_mul: [..., 2] interleaved (re, im), computed in fp32, returned in
// a's dtype.  index_fill: a copy of x with slice `index` of dim set to value.
Tensor complex_mul(const Tensor& a, const Tensor& b);
Tensor index_fill(const Tensor& x, int dim, int64_t index, float value);

Tensor linear_gelu(const Tensor& x, const Tensor& weight, const Tensor& bias);
Tensor linear_silu(const Tensor& x, const Tensor& weight, const Tensor& bias);
Tensor linear_sigmoid(const Tensor& x, const Tensor& weight, const Tensor& bias);

// ---- Fused Roformer entry points (additions the two Roformer models opt
// into; no single reference op matches them).

// One transformer's weights (model_bs_roformer.cu:236-331 names): w_qkv
// [3*H*Dh, dim], w_gate [H, dim], b_gate [H], w_out [dim, H*Dh],
// w_ff1 [ff, dim], b_ff1 [ff], w_ff2 [dim, ff], b_ff2 [dim]; gammas [dim].
// final_gamma: MelBandRoformer's per-transformer output norm, or empty.
struct RoformerLayer {
    Tensor attn_gamma, w_qkv, w_gate, b_gate, w_out;
    Tensor ff_gamma, w_ff1, b_ff1, w_ff2, b_ff2;
    Tensor final_gamma;
};

// The depth loop of model_bs_roformer.cu:482-539 / model_mel_band_roformer.cu:
// 843-906 on x [B, T, F, dim] fp32, in place: layers alternate time and
// frequency transformers (2 * depth entries); final_gamma (BSRoformer's
// output norm) may be empty.  Matrices must all be fp16 or all fp32.
void roformer_stack(Tensor& x, const std::vector<RoformerLayer>& layers, int heads,
                    int dim_head, const Tensor& final_gamma);

// The depth loop's other configurations (model_bs_roformer.cu:477-487,
// :531-535, the apply_transformer loop :319): each depth runs time_depth
// time-axis layers then freq_depth frequency-axis layers (layers holds
// depth * (time_depth + freq_depth) entries in that order, the
// MelBandRoformer norm on the last layer of each transformer), and with
// skip_connection x += sum of the previous depths' outputs before every
// depth after the first.
struct StackSchedule {
    int time_depth = 1;
    int freq_depth = 1;
    bool skip_connection = false;
};
void roformer_stack(Tensor& x, const std::vector<RoformerLayer>& layers, int heads,
                    int dim_head, const Tensor& final_gamma, const StackSchedule& schedule);

// ---- Band split and mask estimator (model_bs_roformer.cu:337-414,
// model_mel_band_roformer.cu:658-738) as grouped launches over all bands.
// band_dims[b] = 2 * freqs_in_band * audio_channels (the reference's
// band_freq_dims_).  Weights per band as the models hold them
// (model_bs_roformer.h:65-70, :105-115): gamma [fd] and W [dim, fd], b [dim]
// for the split; w[b][l] / bias[b][l] for the L linears of band b's MLP.
// fp16 matrices run the grouped kernels (bands.hip); fp32 matrices (the
// reference's fp32 mode) run the reference's per-band loop on the fp32 ops
// (rms_norm, linear, tanh_act, glu), one band at a time.  Gammas and biases
// may be fp16 or fp32.
struct BandSplitWeights {
    std::vector<Tensor> gamma, w, b;
};
struct MaskEstimatorWeights {
    std::vector<std::vector<Tensor>> w, b;  // [band][layer]
};

// The STFT side of the bands: channels (1/2), STFT bins F, and the
// interleaved bin (f * channels + s) of every band feature pair
// (MelBandRoformer's freq_indices_, model_mel_band_roformer.cu:238-268);
// empty freq_indices = every bin once, in order (BSRoformer).
struct StftBands {
    int channels = 0;
    int stft_bins = 0;
    std::vector<int> freq_indices;
};

class BandPlan {
public:
    // Either weight set may be null.  The tensors must outlive the plan.
    BandPlan(std::vector<int> band_dims, int dim, const BandSplitWeights* split,
             const MaskEstimatorWeights* mask, const StftBands* stft = nullptr);
    // STFT [B * ch, F, T, 2] -> band-split input [B, T, sum(band_dims)]
    // (stereo merge, index_select, permute; model_bs_roformer.cu:450-469).
    Tensor band_gather(const Tensor& stft, int64_t batch) const;
    // Stem masks [stems, B, T, sum(band_dims)] and the STFT -> masked STFT
    // [B * stems * ch, F, T, 2] for the iSTFT (scatter_add mean, complex_mul,
    // stereo split, zero DC; model_mel_band_roformer.cu:924-1015).
    Tensor mask_merge(const Tensor& masks, const Tensor& stft, int64_t batch,
                      bool zero_dc) const;
    // x [..., sum(band_dims)] fp32 -> [..., num_bands, dim] fp32
    // (apply_band_split: split, rms_norm * sqrt(fd), linear, stack).
    Tensor band_split(const Tensor& x) const;
    // x [..., num_bands, dim] -> [..., sum(band_dims)] fp32
    // (apply_mask_estimator: per-band MLP with tanh, glu, cat).
    Tensor mask_estimator(const Tensor& x) const;

private:
    std::vector<int> dims_;
    int dim_ = 0, hidden_ = 0, linears_ = 1;
    StftBands stft_;
    bool fp32_ = false;                 // per-band fp32 path
    BandSplitWeights split32_;          // fp32 path: the caller's tensors
    MaskEstimatorWeights mask32_;
    Tensor plan_;
    std::vector<Tensor> keep_;  // fp32 copies of fp16 gammas / biases
    msst_band_config config() const;
};

}  // namespace ops
}  // namespace cudasep
