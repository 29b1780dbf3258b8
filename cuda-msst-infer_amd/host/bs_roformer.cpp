// bs_roformer.cpp — see bs_roformer.h.
#include "bs_roformer.h"

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

// model_bs_roformer.cu:95-190 (load) with the weight names it reads.
void BSRoformer::load(const ModelWeights& weights) {
    cfg_ = BSRConfig::from_json(weights.config());
    const int ch = audio_channels();
    const int nb = (int)cfg_.freqs_per_bands.size();
    if (nb == 0) throw std::runtime_error("BSRoformer: config has no freqs_per_bands");
    const int bins = std::accumulate(cfg_.freqs_per_bands.begin(), cfg_.freqs_per_bands.end(), 0);
    if (bins != cfg_.stft_n_fft / 2 + 1)
        throw std::runtime_error("BSRoformer: freqs_per_bands must cover n_fft / 2 + 1 bins");
    if (cfg_.time_transformer_depth != 1 || cfg_.freq_transformer_depth != 1 || cfg_.skip_connection)
        throw std::runtime_error(
            "BSRoformer: only time/freq_transformer_depth 1 without skip connections is built");
    if (cfg_.stft_win_length != cfg_.stft_n_fft)
        throw std::runtime_error("BSRoformer: stft_win_length must equal stft_n_fft");
    band_dims_.clear();
    for (int f : cfg_.freqs_per_bands) band_dims_.push_back(2 * f * ch);

    window_ = ops::hann_window(cfg_.stft_win_length);

    // band_split.to_features.{b}.{0.gamma, 1.weight, 1.bias}
    split_w_ = ops::BandSplitWeights{};
    for (int b = 0; b < nb; ++b) {
        const std::string p = "band_split.to_features." + std::to_string(b);
        split_w_.gamma.push_back(weights.get(p + ".0.gamma"));
        split_w_.w.push_back(weights.get(p + ".1.weight"));
        split_w_.b.push_back(weights.get(p + ".1.bias"));
    }
    // layers.{d}.{0 time, 1 freq}.layers.0.{0 attention, 1 feed-forward}
    layers_.clear();
    for (int d = 0; d < cfg_.depth; ++d)
        for (int t = 0; t < 2; ++t) {
            const std::string p = "layers." + std::to_string(d) + "." + std::to_string(t) +
                                  ".layers.0";
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
            layers_.push_back(L);
        }
    final_norm_gamma_ = weights.get("final_norm.gamma");
    // mask_estimators.{s}.to_freqs.{b}.0.{2 i}.{weight, bias}, i < mask_estimator_depth
    mask_w_.assign(cfg_.num_stems, ops::MaskEstimatorWeights{});
    for (int s = 0; s < cfg_.num_stems; ++s)
        for (int b = 0; b < nb; ++b) {
            std::vector<Tensor> wl, bl;
            for (int i = 0; i < cfg_.mask_estimator_depth; ++i) {
                const std::string p = "mask_estimators." + std::to_string(s) + ".to_freqs." +
                                      std::to_string(b) + ".0." + std::to_string(2 * i);
                wl.push_back(weights.get(p + ".weight"));
                bl.push_back(weights.get(p + ".bias"));
            }
            mask_w_[s].w.push_back(wl);
            mask_w_[s].b.push_back(bl);
        }

    ops::StftBands sb;
    sb.channels = ch;
    sb.stft_bins = cfg_.stft_n_fft / 2 + 1;
    plans_.clear();
    plans_.emplace_back(new ops::BandPlan(band_dims_, cfg_.dim, &split_w_, &mask_w_[0], &sb));
    for (int s = 1; s < cfg_.num_stems; ++s)
        plans_.emplace_back(new ops::BandPlan(band_dims_, cfg_.dim, nullptr, &mask_w_[s]));
}

// model_bs_roformer.cu:420-609.
Tensor BSRoformer::forward(const Tensor& audio) {
    Tensor a = audio.ndim() == 2 ? audio.unsqueeze(1) : audio;
    if (a.ndim() != 3 || a.dtype() != DType::Float32)
        throw std::runtime_error("BSRoformer::forward: audio must be fp32 [B, channels, samples]");
    const int64_t B = a.size(0), ch = a.size(1), S = a.size(2);
    if (ch != audio_channels())
        throw std::runtime_error("BSRoformer::forward: the model expects " +
                                 std::to_string(audio_channels()) + " channels");
    const int stems = cfg_.num_stems;
    Tensor spec = ops::stft(a.reshape({B * ch, S}), cfg_.stft_n_fft, cfg_.stft_hop_length,
                            cfg_.stft_win_length, window_, true, cfg_.stft_normalized);
    const int64_t T = spec.size(2);
    Tensor feats = plans_[0]->band_split(plans_[0]->band_gather(spec, B));  // [B, T, nb, dim]
    ops::roformer_stack(feats, layers_, cfg_.heads, cfg_.dim_head, final_norm_gamma_);
    int64_t ftot = 0;
    for (int d : band_dims_) ftot += d;
    Tensor masks = Tensor::empty({(int64_t)stems, B, T, ftot});
    for (int s = 0; s < stems; ++s) {
        Tensor m = plans_[s]->mask_estimator(feats);  // [B, T, ftot]
        HIP_CHECK(hipMemcpyAsync(masks.data_f32() + (int64_t)s * B * T * ftot, m.data_f32(),
                                 m.nbytes(), hipMemcpyDeviceToDevice,
                                 CudaContext::instance().stream()));
    }
    Tensor merged = plans_[0]->mask_merge(masks, spec, B, cfg_.zero_dc);  // [B*stems*ch, F, T, 2]
    Tensor recon = ops::istft(merged, cfg_.stft_n_fft, cfg_.stft_hop_length, cfg_.stft_win_length,
                              window_, cfg_.match_input_audio_length ? S : -1, true,
                              cfg_.stft_normalized);
    const int64_t n = recon.size(1);
    return stems == 1 ? recon.reshape({B, ch, n}) : recon.reshape({B, (int64_t)stems, ch, n});
}

}  // namespace cudasep
