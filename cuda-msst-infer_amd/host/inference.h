// inference.h — the chunked inference driver and WAV I/O of the reference's
// cudasep_infer (src/inference_app.{h,cpp}, src/audio_io.{h,cpp}), for the
// BSRoformer and MelBandRoformer models built here.
//
// process_chunked (inference_app.cpp:100-324, "Generic" mode): the mix is
// reflect-padded by border = chunk - step, cut into chunks every `step`
// samples (the last one reflect-padded if it holds more than half a chunk,
// else zero-padded), run through the model `chunk_batch` chunks at a time,
// and overlap-added with linear fades of chunk / 10 samples (no fade at the
// two ends of the track), then divided by the summed fades.  The chunk cut,
// overlap-add and normalisation are device kernels applied in stream order
// (msst_chunk_extract / msst_overlap_add / msst_normalize_by_weights).
#pragma once

#include <functional>
#include <memory>
#include <string>
#include <vector>

#include "roformer_models.h"
#include "tensor.h"
#include "weights.h"

namespace cudasep {
namespace app {

struct AudioData {
    std::vector<float> samples;  // planar [channels][frames]
    int channels = 0;
    int64_t frames = 0;
    int sample_rate = 0;
};

// RIFF/WAVE: PCM 16/24/32-bit or IEEE float 32/64 (also WAVE_FORMAT_EXTENSIBLE).
AudioData load_wav(const std::string& path);
// 32-bit float WAV (audio_io.cpp:280-340); samples planar [channels][frames].
void save_wav(const std::string& path, const float* planar, int channels, int64_t frames,
              int sample_rate);

// inference_app.cpp:59-70: (0, 1) -> overlap ratio; >= 1 -> number of
// overlaps; otherwise the model default.
int resolve_step(int chunk_size, float overlap, int default_overlap);

// audio [channels, S] fp32 on the device -> the model output per chunk
// stitched back to [out_channels, S] (out_channels = stems * channels).
Tensor process_chunked(const Tensor& audio, int chunk_size, int step, int chunk_batch,
                       const std::function<Tensor(const Tensor&)>& forward);

// inference_app.h (ModelType) and inference_app.cpp:77-98: model_type
// names first, then the config keys each family carries.  MDX23C and
// HTDemucs are recognised but not built here (load_model throws).
enum class ModelType { Unknown, MelBandRoformer, BSRoformer, MDX23C, HTDemucs };
ModelType detect_model_type(const JsonValue& config);
const char* model_type_name(ModelType t);

struct LoadedModel {
    ModelWeights weights;
    ModelType type = ModelType::Unknown;
    std::unique_ptr<RoformerModel> model;
    int num_sources = 1;
    int sample_rate = 44100;
    int chunk_size = 0;
    int num_overlap = 2;
    int chunk_batch_size = 2;
    std::vector<std::string> stem_names;
};

// inference_app.cpp:363-447 for BSRoformer and MelBandRoformer checkpoints
// (other model types throw).  quantize_fp16: the reference's --fp16 load.
LoadedModel load_model(const std::string& path, bool quantize_fp16);

// [stems, channels, S] (or [channels, S] for one stem) fp32 on the device.
Tensor run_inference(LoadedModel& model, const AudioData& audio, float overlap);

}  // namespace app
}  // namespace cudasep
