// inference.cpp — see inference.h.
#include "inference.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <fstream>
#include <stdexcept>

#include "msst_hip.h"
#include "ops.h"

namespace cudasep {
namespace app {
namespace {

void check(int rc, const char* what) {
    if (rc != MSST_OK) throw std::runtime_error(std::string(what) + ": " + msst_last_error());
}
hipStream_t stream() { return CudaContext::instance().stream(); }

uint32_t rd32(const unsigned char* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
uint16_t rd16(const unsigned char* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

}  // namespace

AudioData load_wav(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("load_wav: cannot open " + path);
    std::vector<unsigned char> b((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    if (b.size() < 12 || std::memcmp(b.data(), "RIFF", 4) != 0 || std::memcmp(b.data() + 8, "WAVE", 4) != 0)
        throw std::runtime_error("load_wav: not a RIFF/WAVE file " + path);
    int fmt = 0, ch = 0, bits = 0, sr = 0;
    const unsigned char* data = nullptr;
    size_t data_len = 0;
    for (size_t p = 12; p + 8 <= b.size();) {
        const uint32_t len = rd32(&b[p + 4]);
        const unsigned char* body = &b[p + 8];
        const size_t avail = std::min<size_t>(len, b.size() - p - 8);
        if (std::memcmp(&b[p], "fmt ", 4) == 0 && avail >= 16) {
            fmt = rd16(body);
            ch = rd16(body + 2);
            sr = (int)rd32(body + 4);
            bits = rd16(body + 14);
            if (fmt == 0xFFFE && avail >= 26) fmt = rd16(body + 24);  // extensible: SubFormat
        } else if (std::memcmp(&b[p], "data", 4) == 0) {
            data = body;
            data_len = avail;
        }
        p += 8 + len + (len & 1);
    }
    if (!data || ch < 1) throw std::runtime_error("load_wav: no fmt/data chunk in " + path);
    if (!((fmt == 1 && (bits == 16 || bits == 24 || bits == 32)) ||
          (fmt == 3 && (bits == 32 || bits == 64))))
        throw std::runtime_error("load_wav: unsupported format " + std::to_string(fmt) + "/" +
                                 std::to_string(bits) + " bits in " + path);
    const int bps = bits / 8;
    AudioData a;
    a.channels = ch;
    a.sample_rate = sr;
    a.frames = (int64_t)(data_len / (size_t)(bps * ch));
    a.samples.resize((size_t)a.frames * ch);
    for (int64_t i = 0; i < a.frames; ++i)
        for (int c = 0; c < ch; ++c) {
            const unsigned char* s = data + ((size_t)i * ch + c) * bps;
            float v;
            if (fmt == 3 && bits == 32) {
                std::memcpy(&v, s, 4);
            } else if (fmt == 3) {
                double d;
                std::memcpy(&d, s, 8);
                v = (float)d;
            } else if (bits == 16) {
                v = (float)(int16_t)rd16(s) / 32768.0f;
            } else if (bits == 24) {
                int32_t x = (int32_t)((uint32_t)s[0] << 8 | (uint32_t)s[1] << 16 | (uint32_t)s[2] << 24) >> 8;
                v = (float)x / 8388608.0f;
            } else {
                v = (float)((double)(int32_t)rd32(s) / 2147483648.0);
            }
            a.samples[(size_t)c * a.frames + i] = v;
        }
    return a;
}

void save_wav(const std::string& path, const float* planar, int channels, int64_t frames,
              int sample_rate) {
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("save_wav: cannot write " + path);
    const uint32_t data_size = (uint32_t)((uint64_t)channels * frames * 4);
    auto u32 = [&](uint32_t v) { f.write(reinterpret_cast<const char*>(&v), 4); };
    auto u16 = [&](uint16_t v) { f.write(reinterpret_cast<const char*>(&v), 2); };
    f.write("RIFF", 4);
    u32(36 + data_size);
    f.write("WAVEfmt ", 8);
    u32(16);
    u16(3);  // IEEE float
    u16((uint16_t)channels);
    u32((uint32_t)sample_rate);
    u32((uint32_t)(sample_rate * channels * 4));
    u16((uint16_t)(channels * 4));
    u16(32);
    f.write("data", 4);
    u32(data_size);
    std::vector<float> row((size_t)channels);
    for (int64_t i = 0; i < frames; ++i) {
        for (int c = 0; c < channels; ++c) row[c] = planar[(size_t)c * frames + i];
        f.write(reinterpret_cast<const char*>(row.data()), (std::streamsize)(4 * channels));
    }
}

int resolve_step(int chunk_size, float overlap, int default_overlap) {
    if (overlap > 0.0f && overlap < 1.0f)
        return std::max(1, (int)std::lround(chunk_size * (1.0f - overlap)));
    int n = default_overlap;
    if (overlap >= 1.0f) n = std::max(1, (int)std::lround(overlap));
    return std::max(1, chunk_size / std::max(1, n));
}

Tensor process_chunked(const Tensor& audio, int chunk_size, int step, int chunk_batch,
                       const std::function<Tensor(const Tensor&)>& forward) {
    if (audio.ndim() != 2 || audio.dtype() != DType::Float32)
        throw std::runtime_error("process_chunked: audio must be fp32 [channels, samples]");
    if (chunk_size < 1 || step < 1) throw std::runtime_error("process_chunked: bad chunk / step");
    const int64_t C = audio.size(0), S = audio.size(1);
    const int fade_size = chunk_size / 10;
    const int border = chunk_size - step;
    const bool padded = S > 2LL * border && border > 0;
    const int64_t pb = padded ? border : 0;
    const int64_t total = S + 2 * pb;
    std::vector<int64_t> starts;
    for (int64_t s = 0; s < total; s += step) starts.push_back(s);
    const int64_t nchunks = (int64_t)starts.size();
    const int batch = (int)std::max<int64_t>(1, std::min<int64_t>(chunk_batch, nchunks));

    // Fades (inference_app.cpp:195-207, :282-295): ramps of fade_size at both
    // ends, none at the start of the first chunk / the end of the last.
    std::vector<float> fade((size_t)chunk_size, 1.0f);
    if (fade_size == 1) {
        fade.front() = 0.0f;
        fade.back() = 0.0f;
    } else {
        for (int i = 0; i < fade_size; ++i) {
            const float alpha = (float)i / (float)(fade_size - 1);
            fade[i] = alpha;
            fade[chunk_size - fade_size + i] = 1.0f - alpha;
        }
    }
    Tensor windows = Tensor::empty({4, (int64_t)chunk_size});  // plain, first, last, first+last
    for (int v = 0; v < 4; ++v) {
        std::vector<float> w = fade;
        if ((v & 1) && fade_size > 0) std::fill(w.begin(), w.begin() + fade_size, 1.0f);
        if ((v & 2) && fade_size > 0) std::fill(w.end() - fade_size, w.end(), 1.0f);
        HIP_CHECK(hipMemcpyAsync(windows.data_f32() + (int64_t)v * chunk_size, w.data(),
                                 4 * (size_t)chunk_size, hipMemcpyHostToDevice, stream()));
        HIP_CHECK(hipStreamSynchronize(stream()));  // w is a host temporary
    }

    Tensor out, wsum;
    int64_t out_ch = 0;
    for (int64_t g0 = 0; g0 < nchunks; g0 += batch) {
        const int gs = (int)std::min<int64_t>(batch, nchunks - g0);
        Tensor in = Tensor::empty({(int64_t)gs, C, (int64_t)chunk_size});
        for (int l = 0; l < gs; ++l) {
            const int64_t start = starts[(size_t)(g0 + l)];
            const int64_t actual = std::min<int64_t>(chunk_size, total - start);
            check(msst_chunk_extract(audio.data_f32(), C, S, pb, start, chunk_size,
                                     actual < chunk_size && 2 * actual > chunk_size ? 1 : 0,
                                     in.data_f32() + (int64_t)l * C * chunk_size, stream()),
                  "chunk_extract");
        }
        Tensor y = forward(in);  // [gs, ..., n]
        const int64_t n = y.size(-1);
        const int64_t per = y.numel() / ((int64_t)gs * n);  // output channels per chunk
        if (out.is_empty()) {
            out_ch = per;
            out = Tensor::zeros({out_ch, total});
            wsum = Tensor::zeros({total});
        } else if (per != out_ch) {
            throw std::runtime_error("process_chunked: model output channels changed");
        }
        for (int l = 0; l < gs; ++l) {
            const int64_t start = starts[(size_t)(g0 + l)];
            const int64_t actual = std::min<int64_t>(chunk_size, total - start);
            const bool first = start == 0, last = start + chunk_size >= total;
            const int v = (first ? 1 : 0) | (last ? 2 : 0);
            check(msst_overlap_add(out.data_f32(), wsum.data_f32(),
                                   y.data_f32() + (int64_t)l * per * n, n,
                                   windows.data_f32() + (int64_t)v * chunk_size, out_ch, total,
                                   start, std::min<int64_t>(actual, n), stream()),
                  "overlap_add");
        }
    }
    check(msst_normalize_by_weights(out.data_f32(), wsum.data_f32(), out_ch, total, stream()),
          "normalize_by_weights");
    if (!padded) return out;
    Tensor res = Tensor::empty({out_ch, S});
    HIP_CHECK(hipMemcpy2DAsync(res.data_f32(), (size_t)S * 4, out.data_f32() + pb,
                               (size_t)total * 4, (size_t)S * 4, (size_t)out_ch,
                               hipMemcpyDeviceToDevice, stream()));
    return res;
}

ModelType detect_model_type(const JsonValue& cfg) {
    if (cfg.has("model_type")) {
        const std::string mt = cfg.get_string("model_type", "");
        if (mt == "mel_band_roformer" || mt == "MelBandRoformer") return ModelType::MelBandRoformer;
        if (mt == "bs_roformer" || mt == "BSRoformer") return ModelType::BSRoformer;
        if (mt == "mdx23c" || mt == "MDX23C" || mt == "tfc_tdf") return ModelType::MDX23C;
        if (mt == "htdemucs" || mt == "HTDemucs") return ModelType::HTDemucs;
    }
    if (cfg.has("nfft") && cfg.has("depth") && cfg.has("growth")) return ModelType::HTDemucs;
    if (cfg.has("num_bands") || cfg.has("mel_scale")) return ModelType::MelBandRoformer;
    if (cfg.has("freqs_per_bands")) return ModelType::BSRoformer;
    if (cfg.has("num_scales") || cfg.has("bottleneck_factor") || cfg.has("num_subbands"))
        return (cfg.has("growth") && cfg.has("depth")) ? ModelType::HTDemucs : ModelType::MDX23C;
    if (cfg.has("dim") && cfg.has("depth") && cfg.has("dim_head")) return ModelType::BSRoformer;
    return ModelType::Unknown;
}

const char* model_type_name(ModelType t) {
    switch (t) {
        case ModelType::MelBandRoformer: return "MelBandRoformer";
        case ModelType::BSRoformer: return "BSRoformer";
        case ModelType::MDX23C: return "MDX23C";
        case ModelType::HTDemucs: return "HTDemucs";
        default: return "Unknown";
    }
}

LoadedModel load_model(const std::string& path, bool quantize_fp16) {
    LoadedModel m;
    m.weights = ModelWeights::load(path);
    const JsonValue& cfg = m.weights.config();
    m.type = detect_model_type(cfg);
    if (m.type == ModelType::Unknown) throw std::runtime_error("Could not detect model type from config");
    if (m.type == ModelType::BSRoformer)
        m.model.reset(new BSRoformer());
    else if (m.type == ModelType::MelBandRoformer)
        m.model.reset(new MelBandRoformer());
    else
        throw std::runtime_error(std::string("load_model: ") + model_type_name(m.type) +
                                 " checkpoints are not supported here (BSRoformer and "
                                 "MelBandRoformer are)");
    g_quantize_fp16 = quantize_fp16;
    if (quantize_fp16) m.weights.convert_linear_weights_to_fp16();
    m.model->load(m.weights);
    m.num_sources = m.model->num_stems();
    m.sample_rate = m.model->sample_rate();
    m.chunk_size = cfg.get_int("chunk_size", m.model->n_fft() * 256);
    // inference_app.cpp:42-57: num_overlap from the config, else 2 for the Roformers.
    m.num_overlap = cfg.has("num_overlap") ? std::max(1, cfg.get_int("num_overlap", 1)) : 2;
    m.chunk_batch_size = 2;
    // inference_app.cpp:336-361: instruments, sources, target_instrument, stem_i.
    for (const char* key : {"instruments", "sources"})
        if (m.stem_names.empty() && cfg.has(key) && cfg[key].is_array())
            for (size_t i = 0; i < cfg[key].size(); ++i) m.stem_names.push_back(cfg[key][i].as_string());
    if (m.stem_names.empty() && cfg.has("target_instrument"))
        m.stem_names.push_back(cfg.get_string("target_instrument", "target"));
    while ((int)m.stem_names.size() < m.num_sources)
        m.stem_names.push_back("stem_" + std::to_string(m.stem_names.size()));
    m.stem_names.resize((size_t)m.num_sources);
    return m;
}

Tensor run_inference(LoadedModel& model, const AudioData& audio, float overlap) {
    Tensor x = Tensor::from_cpu_f32(audio.samples.data(), {(int64_t)audio.channels, audio.frames});
    auto fwd = [&](const Tensor& in) { return model.model->forward(in); };
    if (model.chunk_size > 0 && audio.frames > model.chunk_size) {
        const int step = resolve_step(model.chunk_size, overlap, model.num_overlap);
        Tensor y = process_chunked(x, model.chunk_size, step, model.chunk_batch_size, fwd);
        return model.num_sources == 1
                   ? y
                   : y.reshape({(int64_t)model.num_sources, (int64_t)audio.channels, audio.frames});
    }
    Tensor y = fwd(x.unsqueeze(0));
    return y.squeeze(0);
}

}  // namespace app
}  // namespace cudasep
