// roformer_models.h — BSRoformer and MelBandRoformer inference on the MI355X
// ops (the reference's src/model_bs_roformer.{h,cu} and
// src/model_mel_band_roformer.{h,cu}): the same config keys and defaults,
// weight names and forward, composed from this library's fused pieces:
//
//   audio [B, ch, S] -> stft -> BandPlan::band_gather -> band_split
//     -> roformer_stack (2 * depth transformers; BSR: global final norm,
//        MBR: a norm closing every transformer)
//     -> one mask estimator per stem -> BandPlan::mask_merge -> istft
//     -> [B, stems, ch, S'] ([B, ch, S'] for one stem)
//
// The two models differ in their bands (BSR: consecutive bins from
// freqs_per_bands; MBR: overlapping mel bands, averaged in the merge), the
// transformer norms and the mask MLP depth (BSR: mask_estimator_depth
// linears; MBR: mask_estimator_depth + 1).  Supported:
// time/freq_transformer_depth 1 without skip connections (the released
// configs); other settings throw at load.
#pragma once

#include <memory>
#include <string>
#include <vector>

#include "json.h"
#include "ops.h"
#include "weights.h"

namespace cudasep {

struct BSRConfig {
    int dim = 384;
    int depth = 12;
    bool stereo = true;
    int num_stems = 1;
    int time_transformer_depth = 1;
    int freq_transformer_depth = 1;
    int dim_head = 64;
    int heads = 8;
    int mask_estimator_depth = 1;
    int mlp_expansion_factor = 4;
    bool zero_dc = true;
    int sample_rate = 44100;
    int stft_n_fft = 2048;
    int stft_hop_length = 441;
    int stft_win_length = 2048;
    bool stft_normalized = false;
    bool match_input_audio_length = false;
    int dim_freqs_in = 1025;
    bool skip_connection = false;
    std::vector<int> freqs_per_bands;

    static BSRConfig from_json(const JsonValue& j);  // model_bs_roformer.cu:21-58
};

struct MBRConfig {
    int dim = 384;
    int depth = 6;
    bool stereo = true;
    int num_stems = 1;
    int time_transformer_depth = 1;
    int freq_transformer_depth = 1;
    int num_bands = 60;
    int dim_head = 64;
    int heads = 8;
    int mask_estimator_depth = 2;
    int mlp_expansion_factor = 4;
    bool zero_dc = true;
    int sample_rate = 44100;
    int stft_n_fft = 2048;
    int stft_hop_length = 441;
    int stft_win_length = 2048;
    bool stft_normalized = false;
    bool match_input_audio_length = false;
    int dim_freqs_in = 1025;
    bool skip_connection = false;

    static MBRConfig from_json(const JsonValue& j);  // model_mel_band_roformer.cu:184-208
};

// MelBandRoformer's bands (model_mel_band_roformer.cu:214-308): the HTK mel
// filterbank of ops::mel_filterbank with fb[0][0] and fb[-1][-1] forced to
// 1, thresholded at > 0; freq_indices interleave the channels (bin f of
// channel s is f * channels + s).
struct MelBands {
    std::vector<int> freq_indices;      // [sum over bands of count * channels]
    std::vector<int> freqs_per_band;    // bins per band
};
MelBands compute_mel_bands(int sample_rate, int n_fft, int num_bands, int channels);

class RoformerModel {
public:
    virtual ~RoformerModel() = default;
    virtual void load(const ModelWeights& weights) = 0;
    // audio [B, channels, samples] or [B, samples] fp32.
    Tensor forward(const Tensor& audio);
    int audio_channels() const { return channels_; }
    int num_stems() const { return stems_; }
    int sample_rate() const { return sample_rate_; }
    int n_fft() const { return n_fft_; }

protected:
    int channels_ = 2, stems_ = 1, sample_rate_ = 44100;
    int n_fft_ = 2048, hop_ = 441, win_length_ = 2048;
    bool normalized_ = false, zero_dc_ = true, match_length_ = false;
    int dim_ = 384, heads_ = 8, dim_head_ = 64;
    std::vector<int> band_dims_;        // 2 * bins * channels per band
    std::vector<int> freq_indices_;     // empty: every bin once, in order
    Tensor window_;
    std::vector<ops::RoformerLayer> layers_;  // per depth: time_depth, then freq_depth layers
    ops::StackSchedule schedule_;
    Tensor final_norm_gamma_;           // BSRoformer only
    ops::BandSplitWeights split_w_;
    std::vector<ops::MaskEstimatorWeights> mask_w_;
    std::vector<std::unique_ptr<ops::BandPlan>> plans_;  // [0]: split + STFT side + stem 0

    // Shared loading steps (the two models use the same weight names for
    // these parts).
    void load_common(const ModelWeights& w, int depth, int time_depth, int freq_depth,
                     bool skip_connection, int linears, bool transformer_norms);
};

class BSRoformer : public RoformerModel {
public:
    void load(const ModelWeights& weights) override;  // model_bs_roformer.cu:95-190
    const BSRConfig& config() const { return cfg_; }

private:
    BSRConfig cfg_;
};

class MelBandRoformer : public RoformerModel {
public:
    void load(const ModelWeights& weights) override;  // model_mel_band_roformer.cu:310-480
    const MBRConfig& config() const { return cfg_; }

private:
    MBRConfig cfg_;
};

}  // namespace cudasep
