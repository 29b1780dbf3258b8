// Host-only check (no GPU) of the MelBandRoformer band construction the
// model loader runs: ops::mel_filterbank_host against the oracle's
// orc_mel_filterbank (same float steps, ops_misc.cu:469-525), and
// compute_mel_bands (corners forced to 1, > 0, channel interleave;
// model_mel_band_roformer.cu:214-308) against bands derived here from the
// oracle's filterbank.  Prints one line per case and "OK" at the end.
#include <cmath>
#include <cstdio>
#include <vector>

#include "msst_oracle.h"
#include "roformer_models.h"

using namespace cudasep;

static int check(int sr, int n_fft, int n_mels, float fmin, float fmax, int ch) {
    const int F = n_fft / 2 + 1;
    const std::vector<float> fb = ops::mel_filterbank_host(sr, n_fft, n_mels, fmin, fmax);
    std::vector<float> ref((size_t)n_mels * F);
    orc_mel_filterbank(ref.data(), sr, n_fft, n_mels, fmin, fmax);
    float worst = 0.0f;
    for (size_t i = 0; i < ref.size(); ++i) worst = std::fmax(worst, std::fabs(fb[i] - ref[i]));
    int bad = fb.size() != ref.size() || worst > 0.0f;
    int nidx = 0;
    if (fmin == 0.0f && fmax == 0.0f) {
        ref[0] = 1.0f;
        ref[(size_t)(n_mels - 1) * F + F - 1] = 1.0f;
        std::vector<int> idx, cnt;
        for (int b = 0; b < n_mels; ++b) {
            int c = 0;
            for (int f = 0; f < F; ++f)
                if (ref[(size_t)b * F + f] > 0.0f) {
                    for (int s = 0; s < ch; ++s) idx.push_back(f * ch + s);
                    ++c;
                }
            cnt.push_back(c);
        }
        const MelBands mb = compute_mel_bands(sr, n_fft, n_mels, ch);
        bad |= mb.freq_indices != idx || mb.freqs_per_band != cnt;
        nidx = (int)mb.freq_indices.size();
    }
    std::printf("sr %d n_fft %d n_mels %d fmin %g fmax %g ch %d: max |diff| %g, %d indices%s\n", sr,
                n_fft, n_mels, fmin, fmax, ch, worst, nidx, bad ? "  MISMATCH" : "");
    return bad;
}

int main() {
    int bad = 0;
    bad += check(44100, 2048, 60, 0.0f, 0.0f, 2);
    bad += check(44100, 2048, 60, 0.0f, 0.0f, 1);
    bad += check(44100, 256, 16, 0.0f, 0.0f, 2);
    bad += check(48000, 1024, 40, 0.0f, 0.0f, 2);
    bad += check(16000, 512, 10, 50.0f, 7000.0f, 2);
    if (bad) return 1;
    std::printf("OK\n");
    return 0;
}
