// msst_infer — separate a WAV file with a BSRoformer or MelBandRoformer .csm
// checkpoint on one MI355X (the file-inference surface of the reference's
// cudasep_infer, src/main.cpp:34-190: same flags and defaults, fp32 weights
// unless --fp16; the HTTP server is not built).
//
//   msst_infer --model m.csm --input mix.wav [--output dir|file.wav]
//              [--stem i|-1] [--overlap f] [--fp16|--fp32]
//              [--chunk-batch-size n] [--device d] [--list-stems]
#include <chrono>
#include <filesystem>
#include <iostream>
#include <string>

#include "inference.h"

namespace fs = std::filesystem;
using namespace cudasep;

namespace {

struct Args {
    std::string model, input, output = "output";
    int stem = 0, device = 0, chunk_batch = 0;
    float overlap = 0.0f;
    bool fp16 = false, list_stems = false;
};

void usage(const char* prog) {
    std::cout << "Usage:\n  " << prog << " --model <path.csm> --input <audio.wav> [options]\n\n"
              << "  --model, -m <path>     .csm model weights\n"
              << "  --input, -i <path>     input WAV (PCM 16/24/32 or float)\n"
              << "  --output, -o <path>    output directory or .wav path (default: output)\n"
              << "  --stem, -s <int>       stem to write (default 0, -1 for all)\n"
              << "  --overlap <float>      (0,1) overlap ratio, >= 1 number of overlaps\n"
              << "  --fp16 / --fp32        fp16 weights with fp32 accumulation / fp32 (default)\n"
              << "  --chunk-batch-size <n> chunks per forward (default 2)\n"
              << "  --device, -d <int>     GPU index (default 0)\n"
              << "  --list-stems           print the model's stems and exit\n";
}

Args parse(int argc, char** argv) {
    Args a;
    for (int i = 1; i < argc; ++i) {
        const std::string s = argv[i];
        auto next = [&]() -> std::string {
            if (i + 1 >= argc) throw std::runtime_error("missing value for " + s);
            return argv[++i];
        };
        if (s == "--model" || s == "-m") a.model = next();
        else if (s == "--input" || s == "-i") a.input = next();
        else if (s == "--output" || s == "-o") a.output = next();
        else if (s == "--stem" || s == "-s") a.stem = std::stoi(next());
        else if (s == "--overlap") a.overlap = std::stof(next());
        else if (s == "--device" || s == "-d") a.device = std::stoi(next());
        else if (s == "--chunk-batch-size") a.chunk_batch = std::stoi(next());
        else if (s == "--fp16" || s == "--quantize") a.fp16 = true;
        else if (s == "--fp32" || s == "--no-fp16") a.fp16 = false;
        else if (s == "--list-stems") a.list_stems = true;
        else if (s == "--help" || s == "-h") {
            usage(argv[0]);
            std::exit(0);
        } else {
            throw std::runtime_error("unknown argument " + s);
        }
    }
    return a;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const Args a = parse(argc, argv);
        if (a.model.empty() || (a.input.empty() && !a.list_stems)) {
            usage(argv[0]);
            return 2;
        }
        HIP_CHECK(hipSetDevice(a.device));
        app::LoadedModel model = app::load_model(a.model, a.fp16);
        if (a.chunk_batch > 0) model.chunk_batch_size = a.chunk_batch;
        std::cout << "  Model type: " << app::model_type_name(model.type) << "\n"
                  << "  Sources: " << model.num_sources << ", Sample rate: " << model.sample_rate
                  << ", Chunk size: " << model.chunk_size << ", Num overlap: " << model.num_overlap
                  << "\n";
        if (a.list_stems) {
            std::cout << "\nModel has " << model.num_sources << " source(s).\n";
            for (size_t i = 0; i < model.stem_names.size(); ++i)
                std::cout << "  [" << i << "] " << model.stem_names[i] << "\n";
            return 0;
        }
        const app::AudioData audio = app::load_wav(a.input);
        // main.cpp:163-166: a rate mismatch is reported, not resampled.
        if (audio.sample_rate != model.sample_rate)
            std::cerr << "Warning: audio sample rate (" << audio.sample_rate
                      << ") != model sample rate (" << model.sample_rate
                      << "). Results may be incorrect.\n";
        if (audio.channels != model.model->audio_channels())
            throw std::runtime_error("the model expects " +
                                     std::to_string(model.model->audio_channels()) + " channels");
        const auto t0 = std::chrono::steady_clock::now();
        Tensor out = app::run_inference(model, audio, a.overlap);
        CudaContext::instance().sync();
        const double ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
        const std::vector<float> host = out.to_cpu_f32();
        const int64_t frames = out.size(-1);
        const int ch = audio.channels;
        // inference_app.cpp:576-617: a one-source model writes output.wav (or
        // the given .wav path) whatever --stem says; a multi-source model
        // writes every stem for -1 or the chosen one, named by its label.
        fs::path out_path(a.output);
        auto target = [&](const std::string& name) {
            if (out_path.extension() == ".wav") return out_path;
            fs::create_directories(out_path);
            return out_path / (name + ".wav");
        };
        auto write = [&](int s, const fs::path& file) {
            app::save_wav(file.string(), host.data() + (size_t)s * ch * frames, ch, frames,
                          model.sample_rate);
            std::cout << "wrote " << file.string() << "\n";
        };
        if (model.num_sources == 1) {
            write(0, target("output"));
        } else if (a.stem >= 0 && a.stem < model.num_sources) {
            write(a.stem, target(model.stem_names[(size_t)a.stem]));
        } else if (a.stem == -1) {
            fs::create_directories(out_path);
            for (int s = 0; s < model.num_sources; ++s)
                write(s, out_path / (model.stem_names[(size_t)s] + ".wav"));
        } else {
            throw std::runtime_error("Stem index out of range");
        }
        std::cout << "inference " << ms << " ms for " << audio.frames << " samples x " << ch
                  << " channels\n";
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "error: " << e.what() << "\n";
        return 1;
    }
}
