// ops.cpp — cudasep::ops on the MI355X C ABI.  See ops.h for the dtype
// rules; each function cites the reference function it stands in for.
#include "ops.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

#include "memory_pool.h"
#include "msst_hip.h"

namespace cudasep {

bool g_quantize_fp16 = false;
bool g_enable_cuda_graph_attention = true;

void clear_attention_graph_cache() {}

CudaContext& CudaContext::instance() {
    static CudaContext ctx;
    return ctx;
}

void CudaContext::sync() { HIP_CHECK(hipDeviceSynchronize()); }

namespace ops {
namespace {

int abi(DType dt) {
    if (dt == DType::Float32) return MSST_F32;
    if (dt == DType::Float16) return MSST_F16;
    throw std::runtime_error("cudasep::ops: int64 tensors are not supported here");
}

void check(int rc, const char* what) {
    if (rc != MSST_OK) throw std::runtime_error(std::string(what) + ": " + msst_last_error());
}

void* stream() { return CudaContext::instance().stream(); }

// Biases, gammas and RoPE tables are consumed as fp32 (the reference's
// ensure_f32 on them), row-major.
Tensor f32(const Tensor& t) { return t.contiguous().to_f32(); }

std::vector<int64_t> with_last(const std::vector<int64_t>& s, int64_t last) {
    std::vector<int64_t> o = s;
    o.back() = last;
    return o;
}

// Shared GEMM driver: act(x . W^T + b) written as out_dtype.
Tensor gemm(const char* name, const Tensor& xv, const Tensor& wv, const Tensor* bias, int act,
            DType out_dtype) {
    const Tensor x = xv.contiguous(), w = wv.contiguous();
    if (w.ndim() != 2) throw std::runtime_error(std::string(name) + ": weight must be 2-D [out, in]");
    if (x.ndim() < 1) throw std::runtime_error(std::string(name) + ": x must have a last dim");
    const int64_t N = w.size(0), K = w.size(1);
    if (x.size(-1) != K)
        throw std::runtime_error(std::string(name) + ": x " + x.shape_str() + " does not match W " +
                                 w.shape_str());
    Tensor b;
    if (bias) {
        if (bias->numel() != N)
            throw std::runtime_error(std::string(name) + ": bias has " +
                                     std::to_string(bias->numel()) + " elements, W has " +
                                     std::to_string(N) + " rows");
        b = f32(*bias);
    }
    const int64_t M = K > 0 ? x.numel() / K : 0;
    Tensor out = Tensor::empty(with_last(x.shape(), N), out_dtype);
    if (M > 0)
        check(msst_linear(x.data_ptr(), abi(x.dtype()), w.data_ptr(), abi(w.dtype()),
                          bias ? b.data_f32() : nullptr, nullptr, out.data_ptr(), abi(out_dtype),
                          M, K, N, act, stream()),
              name);
    return out;
}

// linear / linear_no_bias: fp16 W -> fp32 out; fp32 W -> x's dtype.
DType plain_out(const Tensor& x, const Tensor& w) {
    return w.dtype() == DType::Float16 ? DType::Float32 : x.dtype();
}
// Fused activations: fp16 when x is fp16, else fp32.
DType act_out(const Tensor& x) { return x.dtype() == DType::Float16 ? DType::Float16 : DType::Float32; }

}  // namespace

// ops_norm.cu:455-491
Tensor rms_norm(const Tensor& xv, const Tensor& gamma, float scale) {
    const Tensor x = xv.contiguous();
    if (x.ndim() < 1) throw std::runtime_error("rms_norm: x must have a last dim");
    const int64_t D = x.size(-1);
    if (gamma.numel() != D)
        throw std::runtime_error("rms_norm: gamma has " + std::to_string(gamma.numel()) +
                                 " elements, rows have " + std::to_string(D));
    Tensor g = f32(gamma);
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    const int64_t rows = D > 0 ? x.numel() / D : 0;
    if (rows > 0)
        check(msst_rms_norm(x.data_ptr(), abi(x.dtype()), g.data_f32(), scale, out.data_ptr(),
                            abi(x.dtype()), rows, D, stream()),
              "rms_norm");
    return out;
}

// ops_stft.cu:286-362
Tensor stft(const Tensor& signal, int n_fft, int hop_length, int win_length,
            const Tensor& window, bool center, bool normalized) {
    if (win_length != n_fft || window.numel() != n_fft)
        throw std::runtime_error("stft: the window must have n_fft samples");
    Tensor sig = f32(signal);
    if (sig.ndim() == 1) sig = sig.reshape({1, sig.size(0)});
    if (sig.ndim() != 2) throw std::runtime_error("stft: signal must be [B, L] or [L]");
    const int64_t B = sig.size(0), L = sig.size(1);
    const int64_t T = msst_stft_frames(L, n_fft, hop_length, center ? 1 : 0);
    if (T < 1) throw std::runtime_error("stft: signal too short or bad n_fft / hop");
    Tensor w = f32(window);
    Tensor out = Tensor::empty({B, (int64_t)n_fft / 2 + 1, T, 2}, DType::Float32);
    check(msst_stft(sig.data_f32(), B, L, n_fft, hop_length, w.data_f32(), center ? 1 : 0,
                    normalized ? 1 : 0, out.data_f32(), stream()),
          "stft");
    return out;
}

// ops_stft.cu:368-491
Tensor istft(const Tensor& complex_spec, int n_fft, int hop_length, int win_length,
             const Tensor& window, int64_t length, bool center, bool normalized) {
    if (win_length != n_fft || window.numel() != n_fft)
        throw std::runtime_error("istft: the window must have n_fft samples");
    Tensor spec = f32(complex_spec);
    if (spec.ndim() != 4 || spec.size(1) != n_fft / 2 + 1 || spec.size(3) != 2)
        throw std::runtime_error("istft: spec must be [B, n_fft/2 + 1, T, 2]");
    const int64_t B = spec.size(0), T = spec.size(2);
    const int64_t n = msst_istft_length(T, n_fft, hop_length, length, center ? 1 : 0);
    if (n < 1) throw std::runtime_error("istft: bad n_fft / hop / length");
    Tensor w = f32(window);
    Tensor out = Tensor::empty({B, n}, DType::Float32);
    const int64_t wsb = msst_istft_workspace(B, T, n_fft);
    Tensor ws = Tensor::empty({std::max<int64_t>((wsb + 3) / 4, 1)}, DType::Float32);
    check(msst_istft(spec.data_f32(), B, T, n_fft, hop_length, w.data_f32(), length,
                     center ? 1 : 0, normalized ? 1 : 0, out.data_f32(), ws.data_ptr(), wsb,
                     stream()),
          "istft");
    return out;
}

// ops_stft.cu:264-280
Tensor hann_window(int size) {
    Tensor out = Tensor::empty({(int64_t)std::max(size, 0)}, DType::Float32);
    if (size > 0) check(msst_hann_window(out.data_f32(), size, stream()), "hann_window");
    return out;
}

// ops_misc.cu:469-525
std::vector<float> mel_filterbank_host(int sr, int n_fft, int n_mels, float fmin, float fmax) {
    if (sr <= 0 || n_fft < 2 || n_mels < 1)
        throw std::invalid_argument("mel_filterbank: need sr > 0, n_fft >= 2, n_mels >= 1");
    if (fmax <= 0.0f) fmax = (float)sr / 2.0f;
    const int bins = n_fft / 2 + 1;
    const auto to_mel = [](float hz) { return 2595.0f * std::log10(1.0f + hz / 700.0f); };
    const auto to_hz = [](float mel) { return 700.0f * (std::pow(10.0f, mel / 2595.0f) - 1.0f); };
    const float m0 = to_mel(fmin), m1 = to_mel(fmax);
    std::vector<float> edge((size_t)n_mels + 2);
    for (int i = 0; i < n_mels + 2; ++i)
        edge[(size_t)i] = to_hz(m0 + (m1 - m0) * (float)i / (float)(n_mels + 1));
    std::vector<float> fb((size_t)n_mels * bins, 0.0f);
    for (int m = 0; m < n_mels; ++m) {
        const float lo = edge[(size_t)m], mid = edge[(size_t)m + 1], hi = edge[(size_t)m + 2];
        for (int f = 0; f < bins; ++f) {
            const float hz = (float)sr * (float)f / (float)n_fft;
            float v = 0.0f;
            if (hz >= lo && hz <= mid) {
                if (mid - lo > 0.0f) v = (hz - lo) / (mid - lo);
            } else if (hz > mid && hz <= hi) {
                if (hi - mid > 0.0f) v = (hi - hz) / (hi - mid);
            }
            fb[(size_t)m * bins + f] = v;
        }
    }
    return fb;
}

Tensor mel_filterbank(int sr, int n_fft, int n_mels, float fmin, float fmax) {
    const std::vector<float> fb = mel_filterbank_host(sr, n_fft, n_mels, fmin, fmax);
    return Tensor::from_cpu_f32(fb.data(), {(int64_t)n_mels, (int64_t)(n_fft / 2 + 1)});
}

// ops_elementwise.cu:84-88, :138
Tensor tanh_act(const Tensor& xv) {
    const Tensor x = xv.contiguous();
    Tensor out = Tensor::empty(x.shape(), x.dtype());
    if (x.numel() > 0)
        check(msst_tanh(x.data_ptr(), out.data_ptr(), abi(x.dtype()), x.numel(), stream()),
              "tanh_act");
    return out;
}

// ops_elementwise.cu:282-299: fp32 product of interleaved (re, im) pairs,
// cast back to a's dtype.
Tensor complex_mul(const Tensor& a, const Tensor& b) {
    if (a.ndim() < 1 || a.size(-1) != 2)
        throw std::runtime_error("complex_mul: last dimension must be 2 (re, im)");
    if (a.shape() != b.shape())
        throw std::runtime_error("complex_mul: shapes " + a.shape_str() + " and " + b.shape_str() +
                                 " differ");
    const Tensor af = f32(a), bf = f32(b);
    Tensor out = Tensor::empty(a.shape(), DType::Float32);
    if (a.numel() > 0)
        check(msst_complex_mul(af.data_f32(), bf.data_f32(), out.data_f32(), a.numel() / 2,
                               stream()),
              "complex_mul");
    return out.to_dtype(a.dtype());
}

// ops_elementwise.cu:503-527: a copy of x with index `index` along dim set
// to value (the fill is a broadcast strided copy into that slice).
Tensor index_fill(const Tensor& x, int dim, int64_t index, float value) {
    const int n = x.ndim();
    const int d = dim < 0 ? dim + n : dim;
    if (d < 0 || d >= n) throw std::out_of_range("index_fill: dim out of range");
    if (index < 0 || index >= x.size(d))
        throw std::out_of_range("index_fill: index " + std::to_string(index) + " out of range");
    Tensor out = x.clone();
    Tensor sl = out.slice(d, index, index + 1);
    sl.copy_from(Tensor::full({1}, value, x.dtype()).expand(sl.shape()));
    return out;
}

// ops_elementwise.cu:345-388 (last dimension)
Tensor glu(const Tensor& xv, int dim) {
    const Tensor x = xv.contiguous();
    const int nd = x.ndim();
    if (nd < 1 || (dim != -1 && dim != nd - 1))
        throw std::runtime_error("glu: only the last dimension is supported");
    const int64_t full = x.size(-1);
    if (full % 2 != 0) throw std::runtime_error("glu: last dimension must be even");
    std::vector<int64_t> shape = x.shape();
    shape.back() = full / 2;
    Tensor out = Tensor::empty(shape, x.dtype());
    const int64_t rows = full > 0 ? x.numel() / full : 0;
    if (rows > 0 && full > 0)
        check(msst_glu(x.data_ptr(), out.data_ptr(), abi(x.dtype()), rows, full / 2, stream()),
              "glu");
    return out;
}

// ops_linear.cu:150-343
Tensor linear(const Tensor& x, const Tensor& weight, const Tensor& bias) {
    return gemm("linear", x, weight, &bias, MSST_ACT_NONE, plain_out(x, weight));
}

// ops_linear.cu:349-427
Tensor linear_no_bias(const Tensor& x, const Tensor& weight) {
    return gemm("linear_no_bias", x, weight, nullptr, MSST_ACT_NONE, plain_out(x, weight));
}

// ops_fused.cu:264-282
Tensor linear_gelu(const Tensor& x, const Tensor& weight, const Tensor& bias) {
    return gemm("linear_gelu", x, weight, &bias, MSST_ACT_GELU, act_out(x));
}

// ops_fused.cu:341-358
Tensor linear_silu(const Tensor& x, const Tensor& weight, const Tensor& bias) {
    return gemm("linear_silu", x, weight, &bias, MSST_ACT_SILU, act_out(x));
}

// ops_fused.cu:285-303
Tensor linear_sigmoid(const Tensor& x, const Tensor& weight, const Tensor& bias) {
    return gemm("linear_sigmoid", x, weight, &bias, MSST_ACT_SIGMOID, act_out(x));
}

// ops_attention.cu:522-599 (fused flash attention instead of the
// materialised QK^T / softmax / PV pipeline).
Tensor scaled_dot_product_attention(const Tensor& q, const Tensor& k, const Tensor& v,
                                    float scale, float /*dropout*/) {
    if (q.ndim() != 4 || k.ndim() != 4 || v.ndim() != 4)
        throw std::runtime_error("scaled_dot_product_attention: q, k, v must be 4-D [B,H,N,D]");
    const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3), Nk = k.size(2);
    if (k.size(0) != B || k.size(1) != H || k.size(3) != D || v.size(0) != B ||
        v.size(1) != H || v.size(2) != Nk || v.size(3) != D)
        throw std::runtime_error("scaled_dot_product_attention: shapes q " + q.shape_str() +
                                 ", k " + k.shape_str() + ", v " + v.shape_str() +
                                 " do not agree");
    // One element type for the kernel: k and v follow q.
    const Tensor qc = q.contiguous();
    const Tensor kc = k.contiguous().to_dtype(q.dtype()), vc = v.contiguous().to_dtype(q.dtype());
    Tensor out = Tensor::empty(q.shape(), q.dtype());
    check(msst_attention(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(),
                         abi(q.dtype()), B, H, N, Nk, D, scale, stream()),
          "scaled_dot_product_attention");
    return out;
}

// ops_misc.cu:73-131 (in place; the fp16 path rotates in fp32 registers and
// writes fp16 back, without the reference's f32 round trip tensors).
void apply_rotary_emb(Tensor& q, Tensor& k, const Tensor& cos_freqs, const Tensor& sin_freqs) {
    if (q.ndim() != 4 || k.ndim() != 4)
        throw std::runtime_error("apply_rotary_emb: q and k must be 4-D [B,H,N,D]");
    if (q.shape() != k.shape() || q.dtype() != k.dtype())
        throw std::runtime_error("apply_rotary_emb: q and k must share shape and dtype");
    const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
    if (cos_freqs.numel() < N * (D / 2) || sin_freqs.numel() < N * (D / 2))
        throw std::runtime_error("apply_rotary_emb: cos/sin tables smaller than [N, D/2]");
    Tensor c = f32(cos_freqs), s = f32(sin_freqs);
    // In place; views are rotated through row-major copies written back.
    Tensor qc = q.contiguous(), kc = k.contiguous();
    check(msst_rope_qk(qc.data_ptr(), kc.data_ptr(), abi(q.dtype()), c.data_f32(), s.data_f32(), B,
                       H, N, D, stream()),
          "apply_rotary_emb");
    if (qc.data_ptr() != q.data_ptr()) q.copy_from(qc);
    if (kc.data_ptr() != k.data_ptr()) k.copy_from(kc);
}

// model_bs_roformer.cu:482-539 / model_mel_band_roformer.cu:843-906
void roformer_stack(Tensor& x, const std::vector<RoformerLayer>& layers, int heads, int dim_head,
                    const Tensor& final_gamma) {
    roformer_stack(x, layers, heads, dim_head, final_gamma, StackSchedule{});
}

// model_bs_roformer.cu:477-539 with time/freq_transformer_depth and
// skip_connection: the fused msst_roformer_stack for the plain schedule,
// else one msst_roformer_stack_layer per transformer layer.  The skip sums
// x += store[0] + ... + store[d-1] run as x += S with S the running sum of
// the stored depth outputs (one extra activation instead of depth of them;
// the same terms, summed in another order).
void roformer_stack(Tensor& x, const std::vector<RoformerLayer>& layers, int heads, int dim_head,
                    const Tensor& final_gamma, const StackSchedule& sched) {
    if (x.ndim() != 4 || x.dtype() != DType::Float32 || !x.is_contiguous())
        throw std::runtime_error("roformer_stack: x must be a contiguous fp32 [B, T, F, dim]");
    const int td = sched.time_depth, fd = sched.freq_depth;
    if (td < 1 || fd < 1) throw std::runtime_error("roformer_stack: transformer depths must be >= 1");
    if (layers.size() % (size_t)(td + fd) != 0)
        throw std::runtime_error("roformer_stack: layers must hold depth * (time_depth + "
                                 "freq_depth) transformer layers");
    msst_stack_desc d{};
    d.batch = x.size(0);
    d.frames = x.size(1);
    d.bands = x.size(2);
    d.dim = x.size(3);
    d.heads = heads;
    d.dim_head = dim_head;
    const int64_t depth = (int64_t)layers.size() / (td + fd);
    d.depth = depth;
    d.ff_dim = layers.empty() ? 4 * d.dim : layers[0].w_ff1.size(0);
    const DType wdt = layers.empty() ? DType::Float32 : layers[0].w_qkv.dtype();
    d.w_dtype = abi(wdt);
    // fp32 copies of the vectors, kept alive for the call.
    std::vector<Tensor> keep;
    std::vector<msst_layer_weights> lw(layers.size());
    auto vec = [&](const Tensor& t) -> const float* {
        if (t.is_empty()) return nullptr;
        keep.push_back(f32(t));
        return keep.back().data_f32();
    };
    keep.reserve(layers.size() * 8 + 1);
    for (size_t i = 0; i < layers.size(); ++i) {
        const RoformerLayer& L = layers[i];
        for (const Tensor* m : {&L.w_qkv, &L.w_gate, &L.w_out, &L.w_ff1, &L.w_ff2})
            if (m->dtype() != wdt || !m->is_contiguous())
                throw std::runtime_error(
                    "roformer_stack: weight matrices must be contiguous and share one dtype");
        lw[i].attn_gamma = vec(L.attn_gamma);
        lw[i].w_qkv = L.w_qkv.data_ptr();
        lw[i].w_gate = L.w_gate.data_ptr();
        lw[i].b_gate = vec(L.b_gate);
        lw[i].w_out = L.w_out.data_ptr();
        lw[i].ff_gamma = vec(L.ff_gamma);
        lw[i].w_ff1 = L.w_ff1.data_ptr();
        lw[i].b_ff1 = vec(L.b_ff1);
        lw[i].w_ff2 = L.w_ff2.data_ptr();
        lw[i].b_ff2 = vec(L.b_ff2);
        lw[i].final_gamma = vec(L.final_gamma);
    }
    const float* fg = vec(final_gamma);
    const int64_t ws = msst_roformer_stack_workspace(&d);
    if (ws < 0) throw std::runtime_error(std::string("roformer_stack: ") + msst_last_error());
    Tensor work = Tensor::empty({ws}, DType::Float16);  // byte buffer (>= ws bytes)
    if (td == 1 && fd == 1 && !sched.skip_connection) {
        check(msst_roformer_stack(x.data_f32(), &d, lw.data(), fg, work.data_ptr(), 2 * ws,
                                  stream()),
              "roformer_stack");
        return;
    }
    Tensor skip_sum;  // sum of the depth outputs stored so far
    size_t li = 0;
    for (int64_t dd = 0; dd < depth; ++dd) {
        if (sched.skip_connection && dd > 0) x.add_(skip_sum);
        for (int t = 0; t < td + fd; ++t, ++li)
            check(msst_roformer_stack_layer(x.data_f32(), &d, &lw[li], t < td ? 0 : 1,
                                            work.data_ptr(), 2 * ws, stream()),
                  "roformer_stack");
        if (sched.skip_connection && dd + 1 < depth) {
            if (dd == 0)
                skip_sum = x.clone();
            else
                skip_sum.add_(x);
        }
    }
    if (fg)
        check(msst_rms_norm(x.data_f32(), MSST_F32, fg, std::sqrt((float)d.dim), x.data_f32(),
                            MSST_F32, x.numel() / d.dim, d.dim, stream()),
              "roformer_stack");
}

// ---------------------------------------------------------------------------
// BandPlan
// ---------------------------------------------------------------------------
msst_band_config BandPlan::config() const {
    msst_band_config c;
    c.num_bands = (int)dims_.size();
    c.band_dims = dims_.data();
    c.dim = dim_;
    c.hidden = hidden_;
    c.mlp_linears = linears_;
    c.audio_channels = stft_.channels;
    c.stft_bins = stft_.stft_bins;
    c.freq_indices = stft_.freq_indices.empty() ? nullptr : stft_.freq_indices.data();
    return c;
}

BandPlan::BandPlan(std::vector<int> band_dims, int dim, const BandSplitWeights* split,
                   const MaskEstimatorWeights* mask, const StftBands* stft)
    : dims_(std::move(band_dims)), dim_(dim) {
    if (stft) stft_ = *stft;
    const size_t nb = dims_.size();
    if (mask) {
        if (mask->w.size() != nb || mask->b.size() != nb || mask->w[0].empty())
            throw std::runtime_error("BandPlan: mask estimator needs weights for every band");
        linears_ = (int)mask->w[0].size();
        hidden_ = linears_ > 1 ? (int)mask->w[0][0].size(0) : 0;
    }
    const msst_band_config c = config();
    const int64_t bytes = msst_band_plan_bytes(&c);
    if (bytes < 0) throw std::runtime_error("BandPlan: unsupported band configuration");
    plan_ = Tensor::empty({(bytes + 3) / 4}, DType::Float32);
    auto f32v = [&](const Tensor& t) -> const float* {
        if (t.dtype() == DType::Float32) return t.data_f32();
        keep_.push_back(t.to_f32());
        return keep_.back().data_f32();
    };
    // fp32 matrices select the per-band fp32 path (all matrices one dtype).
    const Tensor* first = split && !split->w.empty() ? &split->w[0]
                          : mask && !mask->w.empty() && !mask->w[0].empty() ? &mask->w[0][0]
                                                                              : nullptr;
    fp32_ = first && first->dtype() == DType::Float32;
    const DType mdt = fp32_ ? DType::Float32 : DType::Float16;
    auto f16w = [&](const Tensor& t) -> const void* {
        if (t.dtype() != mdt)
            throw std::runtime_error("BandPlan: band matrices must all be fp16 or all fp32");
        return t.data_ptr();
    };
    std::vector<const float*> sg, sb, mb;
    std::vector<const void*> sw, mw;
    if (split) {
        if (split->gamma.size() != nb || split->w.size() != nb || split->b.size() != nb)
            throw std::runtime_error("BandPlan: band split needs weights for every band");
        for (size_t b = 0; b < nb; ++b) {
            if (split->w[b].ndim() != 2 || split->w[b].size(0) != dim ||
                split->w[b].size(1) != dims_[b] || split->gamma[b].numel() != dims_[b] ||
                split->b[b].numel() != dim)
                throw std::runtime_error("BandPlan: band split weight " + std::to_string(b) +
                                         " has the wrong shape");
            sg.push_back(f32v(split->gamma[b]));
            sw.push_back(f16w(split->w[b]));
            sb.push_back(f32v(split->b[b]));
        }
    }
    if (mask) {
        for (size_t b = 0; b < nb; ++b) {
            if ((int)mask->w[b].size() != linears_ || (int)mask->b[b].size() != linears_)
                throw std::runtime_error("BandPlan: every band MLP needs the same depth");
            int64_t K = dim;
            for (int l = 0; l < linears_; ++l) {
                const int64_t N = l == linears_ - 1 ? 2 * dims_[b] : hidden_;
                const Tensor& w = mask->w[b][l];
                if (w.ndim() != 2 || w.size(0) != N || w.size(1) != K ||
                    mask->b[b][l].numel() != N)
                    throw std::runtime_error("BandPlan: mask estimator weight (" +
                                             std::to_string(b) + ", " + std::to_string(l) +
                                             ") has the wrong shape");
                mw.push_back(f16w(w));
                mb.push_back(f32v(mask->b[b][l]));
                K = N;
            }
        }
    }
    if (fp32_) {
        // The plan keeps only the STFT side; the matrices stay with the ops.
        if (split) split32_ = *split;
        if (mask) mask32_ = *mask;
        check(msst_band_plan_init(&c, nullptr, nullptr, nullptr, nullptr, nullptr,
                                  plan_.data_ptr(), bytes, stream()),
              "BandPlan");
        return;
    }
    check(msst_band_plan_init(&c, split ? sg.data() : nullptr, split ? sw.data() : nullptr,
                              split ? sb.data() : nullptr, mask ? mw.data() : nullptr,
                              mask ? mb.data() : nullptr, plan_.data_ptr(), bytes, stream()),
          "BandPlan");
}

namespace {
// dst[r, 0..cols) = src[r * src_pitch + 0..cols) (elements of `bytes_per`).
void copy2d(void* dst, int64_t dst_pitch, const void* src, int64_t src_pitch, int64_t cols,
            int64_t rows, size_t bytes_per) {
    if (rows == 0 || cols == 0) return;
    HIP_CHECK(hipMemcpy2DAsync(dst, (size_t)dst_pitch * bytes_per, src,
                               (size_t)src_pitch * bytes_per, (size_t)cols * bytes_per,
                               (size_t)rows, hipMemcpyDeviceToDevice,
                               reinterpret_cast<hipStream_t>(stream())));
}
}  // namespace

Tensor BandPlan::band_gather(const Tensor& stftv, int64_t batch) const {
    const Tensor stft = stftv.contiguous();
    if (stft_.channels == 0) throw std::runtime_error("band_gather: plan has no STFT side");
    if (stft.ndim() != 4 || stft.dtype() != DType::Float32 || stft.size(3) != 2 ||
        stft.size(0) != batch * stft_.channels || stft.size(1) != stft_.stft_bins)
        throw std::runtime_error("band_gather: stft must be fp32 [batch * channels, F, T, 2]");
    int64_t ftot = 0;
    for (int d : dims_) ftot += d;
    const int64_t T = stft.size(2);
    Tensor out = Tensor::empty({batch, T, ftot}, DType::Float32);
    const msst_band_config c = config();
    check(msst_band_gather(&c, plan_.data_ptr(), stft.data_f32(), batch, T, out.data_f32(),
                           stream()),
          "band_gather");
    return out;
}

Tensor BandPlan::mask_merge(const Tensor& masksv, const Tensor& stftv, int64_t batch,
                            bool zero_dc) const {
    const Tensor masks = masksv.contiguous(), stft = stftv.contiguous();
    if (stft_.channels == 0) throw std::runtime_error("mask_merge: plan has no STFT side");
    int64_t ftot = 0;
    for (int d : dims_) ftot += d;
    if (stft.ndim() != 4 || stft.dtype() != DType::Float32 || stft.size(3) != 2 ||
        stft.size(0) != batch * stft_.channels || stft.size(1) != stft_.stft_bins)
        throw std::runtime_error("mask_merge: stft must be fp32 [batch * channels, F, T, 2]");
    const int64_t T = stft.size(2);
    if (masks.ndim() != 4 || masks.dtype() != DType::Float32 || masks.size(1) != batch ||
        masks.size(2) != T || masks.size(3) != ftot)
        throw std::runtime_error("mask_merge: masks must be fp32 [stems, batch, T, sum(dims)]");
    const int64_t stems = masks.size(0);
    Tensor out = Tensor::empty({batch * stems * stft_.channels, (int64_t)stft_.stft_bins, T, 2},
                               DType::Float32);
    const msst_band_config c = config();
    const int64_t wsb = msst_mask_merge_workspace(&c, batch, stems, T);
    Tensor ws = Tensor::empty({std::max<int64_t>((wsb + 3) / 4, 1)}, DType::Float32);
    check(msst_mask_merge(&c, plan_.data_ptr(), masks.data_f32(), stems, stft.data_f32(), batch,
                          T, zero_dc ? 1 : 0, out.data_f32(), ws.data_ptr(), wsb, stream()),
          "mask_merge");
    return out;
}

Tensor BandPlan::band_split(const Tensor& xv) const {
    const Tensor x = xv.contiguous();
    int64_t ftot = 0;
    for (int d : dims_) ftot += d;
    if (x.ndim() < 1 || x.size(-1) != ftot || x.dtype() != DType::Float32)
        throw std::runtime_error("band_split: x must be fp32 [..., sum(band_dims)]");
    const int64_t rows = x.numel() / ftot;
    std::vector<int64_t> shape = x.shape();
    shape.back() = (int64_t)dims_.size();
    shape.push_back(dim_);
    Tensor out = Tensor::empty(shape, DType::Float32);
    if (fp32_) {
        // model_bs_roformer.cu:337-368, band by band on the fp32 ops.
        if (split32_.w.empty()) throw std::runtime_error("band_split: plan has no split weights");
        const int64_t nb = (int64_t)dims_.size();
        int64_t off = 0;
        for (int64_t b = 0; b < nb; ++b) {
            const int64_t d = dims_[b];
            Tensor xb = Tensor::empty({rows, d});
            copy2d(xb.data_ptr(), d, x.data_f32() + off, ftot, d, rows, 4);
            Tensor o = linear(rms_norm(xb, split32_.gamma[b], std::sqrt((float)d)), split32_.w[b],
                              split32_.b[b]);
            copy2d(out.data_f32() + b * dim_, nb * dim_, o.data_ptr(), dim_, dim_, rows, 4);
            off += d;
        }
        return out;
    }
    const msst_band_config c = config();
    const int64_t wsb = msst_band_split_workspace(&c, rows);
    Tensor ws = Tensor::empty({std::max<int64_t>((wsb + 3) / 4, 1)}, DType::Float32);
    check(msst_band_split(&c, plan_.data_ptr(), x.data_f32(), rows, out.data_f32(), ws.data_ptr(),
                          wsb, stream()),
          "band_split");
    return out;
}

Tensor BandPlan::mask_estimator(const Tensor& xv) const {
    const Tensor x = xv.contiguous();
    const int64_t nb = (int64_t)dims_.size();
    if (x.ndim() < 2 || x.size(-1) != dim_ || x.size(-2) != nb)
        throw std::runtime_error("mask_estimator: x must be [..., num_bands, dim]");
    int64_t ftot = 0;
    for (int d : dims_) ftot += d;
    const int64_t rows = x.numel() / (nb * dim_);
    std::vector<int64_t> shape(x.shape().begin(), x.shape().end() - 2);
    shape.push_back(ftot);
    Tensor out = Tensor::empty(shape, DType::Float32);
    if (fp32_) {
        // model_bs_roformer.cu:374-414, band by band on the fp32 ops.
        if (mask32_.w.empty()) throw std::runtime_error("mask_estimator: plan has no MLP weights");
        Tensor xf = x.to_f32();
        int64_t off = 0;
        for (int64_t b = 0; b < nb; ++b) {
            Tensor h = Tensor::empty({rows, (int64_t)dim_});
            copy2d(h.data_ptr(), dim_, xf.data_f32() + b * dim_, nb * dim_, dim_, rows, 4);
            for (int l = 0; l < linears_; ++l) {
                h = linear(h, mask32_.w[b][l], mask32_.b[b][l]);
                if (l < linears_ - 1) h = tanh_act(h);
            }
            Tensor g = glu(h, -1);
            const int64_t d = dims_[b];
            copy2d(out.data_f32() + off, ftot, g.data_ptr(), d, d, rows, 4);
            off += d;
        }
        return out;
    }
    const msst_band_config c = config();
    const int64_t wsb = msst_mask_estimator_workspace(&c, rows);
    Tensor ws = Tensor::empty({std::max<int64_t>((wsb + 3) / 4, 1)}, DType::Float32);
    check(msst_mask_estimator(&c, plan_.data_ptr(), x.data_ptr(), abi(x.dtype()), rows,
                              out.data_f32(), ws.data_ptr(), wsb, stream()),
          "mask_estimator");
    return out;
}

}  // namespace ops
}  // namespace cudasep
