// roformer_models.cpp — see roformer_models.h.
#include "roformer_models.h"

#include <cmath>
#include <numeric>
#include <stdexcept>

namespace cudasep {

// model_bs_roformer.cu:21-58 (same keys and defaults).
BSRConfig BSRConfig::from_json(const JsonValue& j) {
    BSRConfig c;
    c.dim = j.get_int("dim", c.dim);
    c.depth = j.get_int("depth", c.depth);
    c.stereo = j.get_bool("stereo", c.stereo);
    c.num_stems = j.get_int("num_stems", c.num_stems);
    c.time_transformer_depth = j.get_int("time_transformer_depth", c.time_transformer_depth);
    c.freq_transformer_depth = j.get_int("freq_transformer_depth", c.freq_transformer_depth);
    c.dim_head = j.get_int("dim_head", c.dim_head);
    c.heads = j.get_int("heads", c.heads);
    c.mask_estimator_depth = j.get_int("mask_estimator_depth", c.mask_estimator_depth);
    c.mlp_expansion_factor = j.get_int("mlp_expansion_factor", c.mlp_expansion_factor);
    c.zero_dc = j.get_bool("zero_dc", c.zero_dc);
    c.sample_rate = j.get_int("sample_rate", c.sample_rate);
    c.stft_n_fft = j.get_int("stft_n_fft", c.stft_n_fft);
    c.stft_hop_length = j.get_int("stft_hop_length", c.stft_hop_length);
    c.stft_win_length = j.get_int("stft_win_length", c.stft_win_length);
    c.stft_normalized = j.get_bool("stft_normalized", c.stft_normalized);
    c.match_input_audio_length = j.get_bool("match_input_audio_length", c.match_input_audio_length);
    c.dim_freqs_in = j.get_int("dim_freqs_in", c.dim_freqs_in);
    c.skip_connection = j.get_bool("skip_connection", c.skip_connection);
    if (j.has("freqs_per_bands") && j["freqs_per_bands"].is_array()) {
        const JsonValue& a = j["freqs_per_bands"];
        for (size_t i = 0; i < a.size(); ++i) c.freqs_per_bands.push_back(a[i].as_int());
    }
    return c;
}

// model_mel_band_roformer.cu:184-208 (same keys and defaults).
MBRConfig MBRConfig::from_json(const JsonValue& j) {
    MBRConfig c;
    c.dim = j.get_int("dim", c.dim);
    c.depth = j.get_int("depth", c.depth);
    c.stereo = j.get_bool("stereo", c.stereo);
    c.num_stems = j.get_int("num_stems", c.num_stems);
    c.time_transformer_depth = j.get_int("time_transformer_depth", c.time_transformer_depth);
    c.freq_transformer_depth = j.get_int("freq_transformer_depth", c.freq_transformer_depth);
    c.num_bands = j.get_int("num_bands", c.num_bands);
    c.dim_head = j.get_int("dim_head", c.dim_head);
    c.heads = j.get_int("heads", c.heads);
    c.mask_estimator_depth = j.get_int("mask_estimator_depth", c.mask_estimator_depth);
    c.mlp_expansion_factor = j.get_int("mlp_expansion_factor", c.mlp_expansion_factor);
    c.zero_dc = j.get_bool("zero_dc", c.zero_dc);
    c.sample_rate = j.get_int("sample_rate", c.sample_rate);
    c.stft_n_fft = j.get_int("stft_n_fft", c.stft_n_fft);
    c.stft_hop_length = j.get_int("stft_hop_length", c.stft_hop_length);
    c.stft_win_length = j.get_int("stft_win_length", c.stft_win_length);
    c.stft_normalized = j.get_bool("stft_normalized", c.stft_normalized);
    c.match_input_audio_length = j.get_bool("match_input_audio_length", c.match_input_audio_length);
    c.dim_freqs_in = j.get_int("dim_freqs_in", c.dim_freqs_in);
    c.skip_connection = j.get_bool("skip_connection", c.skip_connection);
    return c;
}

// ops_misc.cu:469-528 (HTK mel scale, triangles in float) and
// model_mel_band_roformer.cu:214-308 (forced corners, > 0, channel interleave).
MelBands compute_mel_bands(int sr, int n_fft, int num_bands, int channels) {
    std::vector<float> fb = ops::mel_filterbank_host(sr, n_fft, num_bands, 0.0f, 0.0f);
    const int bins = n_fft / 2 + 1;
    fb[0] = 1.0f;
    fb[(size_t)(num_bands - 1) * bins + (bins - 1)] = 1.0f;
    MelBands mb;
    for (int b = 0; b < num_bands; ++b) {
        int count = 0;
        for (int f = 0; f < bins; ++f)
            if (fb[(size_t)b * bins + f] > 0.0f) {
                for (int s = 0; s < channels; ++s) mb.freq_indices.push_back(f * channels + s);
                ++count;
            }
        mb.freqs_per_band.push_back(count);
    }
    return mb;
}

void RoformerModel::load_common(const ModelWeights& weights, int depth, int time_depth,
                                int freq_depth, bool skip_connection, int linears,
                                bool transformer_norms) {
    if (depth < 1 || time_depth < 1 || freq_depth < 1)
        throw std::runtime_error("Roformer: depth and transformer depths must be >= 1");
    schedule_ = ops::StackSchedule{time_depth, freq_depth, skip_connection};
    const int nb = (int)band_dims_.size();
    window_ = ops::hann_window(win_length_);
    // band_split.to_features.{b}.{0.gamma, 1.weight, 1.bias}
    split_w_ = ops::BandSplitWeights{};
    for (int b = 0; b < nb; ++b) {
        const std::string p = "band_split.to_features." + std::to_string(b);
        split_w_.gamma.push_back(weights.get(p + ".0.gamma"));
        split_w_.w.push_back(weights.get(p + ".1.weight"));
        split_w_.b.push_back(weights.get(p + ".1.bias"));
    }
    // layers.{d}.{0 time, 1 freq}.layers.{i}.{0 attention, 1 feed-forward},
    // i < the transformer's depth (+ layers.{d}.{t}.norm.gamma closing each
    // MelBandRoformer transformer, after its last layer)
    layers_.clear();
    for (int d = 0; d < depth; ++d)
        for (int t = 0; t < 2; ++t)
            for (int i = 0, n = t == 0 ? time_depth : freq_depth; i < n; ++i) {
                const std::string tp = "layers." + std::to_string(d) + "." + std::to_string(t);
                const std::string p = tp + ".layers." + std::to_string(i);
                ops::RoformerLayer L;
                L.attn_gamma = weights.get(p + ".0.norm.gamma");
                L.w_qkv = weights.get(p + ".0.to_qkv.weight");
                L.w_gate = weights.get(p + ".0.to_gates.weight");
                L.b_gate = weights.get(p + ".0.to_gates.bias");
                L.w_out = weights.get(p + ".0.to_out.0.weight");
                L.ff_gamma = weights.get(p + ".1.net.0.gamma");
                L.w_ff1 = weights.get(p + ".1.net.1.weight");
                L.b_ff1 = weights.get(p + ".1.net.1.bias");
                L.w_ff2 = weights.get(p + ".1.net.4.weight");
                L.b_ff2 = weights.get(p + ".1.net.4.bias");
                if (transformer_norms && i == n - 1) L.final_gamma = weights.get(tp + ".norm.gamma");
                layers_.push_back(L);
            }
    // mask_estimators.{s}.to_freqs.{b}.0.{2 i}.{weight, bias}, i < linears
    mask_w_.assign(stems_, ops::MaskEstimatorWeights{});
    for (int s = 0; s < stems_; ++s)
        for (int b = 0; b < nb; ++b) {
            std::vector<Tensor> wl, bl;
            for (int i = 0; i < linears; ++i) {
                const std::string p = "mask_estimators." + std::to_string(s) + ".to_freqs." +
                                      std::to_string(b) + ".0." + std::to_string(2 * i);
                wl.push_back(weights.get(p + ".weight"));
                bl.push_back(weights.get(p + ".bias"));
            }
            mask_w_[s].w.push_back(wl);
            mask_w_[s].b.push_back(bl);
        }
    ops::StftBands sb;
    sb.channels = channels_;
    sb.stft_bins = n_fft_ / 2 + 1;
    sb.freq_indices = freq_indices_;
    plans_.clear();
    plans_.emplace_back(new ops::BandPlan(band_dims_, dim_, &split_w_, &mask_w_[0], &sb));
    for (int s = 1; s < stems_; ++s)
        plans_.emplace_back(new ops::BandPlan(band_dims_, dim_, nullptr, &mask_w_[s]));
}

void BSRoformer::load(const ModelWeights& weights) {
    cfg_ = BSRConfig::from_json(weights.config());
    channels_ = cfg_.stereo ? 2 : 1;
    stems_ = cfg_.num_stems;
    sample_rate_ = cfg_.sample_rate;
    n_fft_ = cfg_.stft_n_fft;
    hop_ = cfg_.stft_hop_length;
    win_length_ = cfg_.stft_win_length;
    normalized_ = cfg_.stft_normalized;
    zero_dc_ = cfg_.zero_dc;
    match_length_ = cfg_.match_input_audio_length;
    dim_ = cfg_.dim;
    heads_ = cfg_.heads;
    dim_head_ = cfg_.dim_head;
    if (cfg_.freqs_per_bands.empty()) throw std::runtime_error("BSRoformer: config has no freqs_per_bands");
    const int bins = std::accumulate(cfg_.freqs_per_bands.begin(), cfg_.freqs_per_bands.end(), 0);
    if (bins != n_fft_ / 2 + 1)
        throw std::runtime_error("BSRoformer: freqs_per_bands must cover n_fft / 2 + 1 bins");
    if (win_length_ != n_fft_) throw std::runtime_error("BSRoformer: stft_win_length must equal stft_n_fft");
    band_dims_.clear();
    for (int f : cfg_.freqs_per_bands) band_dims_.push_back(2 * f * channels_);
    freq_indices_.clear();
    load_common(weights, cfg_.depth, cfg_.time_transformer_depth, cfg_.freq_transformer_depth,
                cfg_.skip_connection, cfg_.mask_estimator_depth, false);
    final_norm_gamma_ = weights.get("final_norm.gamma");
}

void MelBandRoformer::load(const ModelWeights& weights) {
    cfg_ = MBRConfig::from_json(weights.config());
    channels_ = cfg_.stereo ? 2 : 1;
    stems_ = cfg_.num_stems;
    sample_rate_ = cfg_.sample_rate;
    n_fft_ = cfg_.stft_n_fft;
    hop_ = cfg_.stft_hop_length;
    win_length_ = cfg_.stft_win_length;
    normalized_ = cfg_.stft_normalized;
    zero_dc_ = cfg_.zero_dc;
    match_length_ = cfg_.match_input_audio_length;
    dim_ = cfg_.dim;
    heads_ = cfg_.heads;
    dim_head_ = cfg_.dim_head;
    if (win_length_ != n_fft_)
        throw std::runtime_error("MelBandRoformer: stft_win_length must equal stft_n_fft");
    const int nb = cfg_.num_bands;
    std::vector<int> counts;
    freq_indices_.clear();
    if (weights.has("__precomputed__.freq_indices")) {
        // Bands stored with the checkpoint (model_mel_band_roformer.cu:312-350):
        // int64 freq_indices (channel-interleaved) and per-band bin counts.
        const Tensor& fi = weights.get("__precomputed__.freq_indices");
        const Tensor& nf = weights.get("__precomputed__.num_freqs_per_band");
        if (fi.dtype() != DType::Int64 || nf.dtype() != DType::Int64 || nf.numel() != nb)
            throw std::runtime_error("MelBandRoformer: bad __precomputed__ band tensors");
        std::vector<int64_t> a((size_t)fi.numel()), c((size_t)nb);
        fi.copy_to_cpu(a.data(), a.size() * 8);
        nf.copy_to_cpu(c.data(), c.size() * 8);
        int64_t total = 0;
        for (int64_t v : c) {
            if (v < 1) throw std::runtime_error("MelBandRoformer: a precomputed band has no bins");
            total += v;
            counts.push_back((int)v);
        }
        if (total * channels_ != (int64_t)a.size())
            throw std::runtime_error(
                "MelBandRoformer: __precomputed__.freq_indices does not match num_freqs_per_band");
        const int64_t limit = (int64_t)(n_fft_ / 2 + 1) * channels_;
        for (int64_t v : a) {
            if (v < 0 || v >= limit)
                throw std::runtime_error("MelBandRoformer: precomputed frequency index out of range");
            freq_indices_.push_back((int)v);
        }
    } else {
        const MelBands mb = compute_mel_bands(sample_rate_, n_fft_, nb, channels_);
        freq_indices_ = mb.freq_indices;
        counts = mb.freqs_per_band;
        for (int cnt : counts)
            if (cnt < 1) throw std::runtime_error("MelBandRoformer: a mel band holds no STFT bin");
    }
    band_dims_.clear();
    for (int cnt : counts) band_dims_.push_back(2 * cnt * channels_);
    load_common(weights, cfg_.depth, cfg_.time_transformer_depth, cfg_.freq_transformer_depth,
                cfg_.skip_connection, cfg_.mask_estimator_depth + 1, true);
    final_norm_gamma_ = Tensor();
}

// model_bs_roformer.cu:420-609 / model_mel_band_roformer.cu:745-1040.
Tensor RoformerModel::forward(const Tensor& audio) {
    Tensor a = audio.ndim() == 2 ? audio.unsqueeze(1) : audio;
    if (a.ndim() != 3 || a.dtype() != DType::Float32)
        throw std::runtime_error("Roformer forward: audio must be fp32 [B, channels, samples]");
    const int64_t B = a.size(0), ch = a.size(1), S = a.size(2);
    if (ch != channels_)
        throw std::runtime_error("Roformer forward: the model expects " + std::to_string(channels_) +
                                 " channels");
    Tensor spec = ops::stft(a.reshape({B * ch, S}), n_fft_, hop_, win_length_, window_, true,
                            normalized_);
    const int64_t T = spec.size(2);
    Tensor feats = plans_[0]->band_split(plans_[0]->band_gather(spec, B));  // [B, T, nb, dim]
    ops::roformer_stack(feats, layers_, heads_, dim_head_, final_norm_gamma_, schedule_);
    int64_t ftot = 0;
    for (int d : band_dims_) ftot += d;
    Tensor masks = Tensor::empty({(int64_t)stems_, B, T, ftot});
    for (int s = 0; s < stems_; ++s) {
        Tensor m = plans_[s]->mask_estimator(feats);  // [B, T, ftot]
        HIP_CHECK(hipMemcpyAsync(masks.data_f32() + (int64_t)s * B * T * ftot, m.data_f32(),
                                 m.nbytes(), hipMemcpyDeviceToDevice,
                                 CudaContext::instance().stream()));
    }
    Tensor merged = plans_[0]->mask_merge(masks, spec, B, zero_dc_);  // [B*stems*ch, F, T, 2]
    Tensor recon = ops::istft(merged, n_fft_, hop_, win_length_, window_, match_length_ ? S : -1,
                              true, normalized_);
    const int64_t n = recon.size(1);
    return stems_ == 1 ? recon.reshape({B, ch, n}) : recon.reshape({B, (int64_t)stems_, ch, n});
}

}  // namespace cudasep
