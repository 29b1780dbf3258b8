// stft.hip — STFT / iSTFT with a hand-written LDS FFT (the reference calls
// cuFFT, ops_stft.cu:286-491).  Semantics are the reference's (torch.stft /
// torch.istft): centre reflect padding, the caller's window (length n_fft),
// onesided [B, n_fft/2 + 1, T, 2] spectra, optional 1/sqrt(n_fft) scaling,
// and an inverse that overlap-adds the windowed frames and divides by the
// summed squared window where it exceeds 1e-8.
//
//   stft_kernel         one workgroup per (frame, signal): gather the frame
//                       (reflect padding computed from the index), window
//                       it, pack the 2M real samples into M complex ones, an
//                       M-point Stockham FFT in LDS, unpack to the M + 1
//                       bins (fft_core.hpp).
//   istft_frame_kernel  one workgroup per (frame, signal): the inverse of the
//                       above (pack the bins, FFT of the conjugate, conjugate
//                       and 1/M), windowed, to a frame buffer.
//   istft_ola_kernel    one thread per output sample: sums the <= ceil(n_fft /
//                       hop) frames that cover it in frame order (the
//                       reference uses atomicAdd, whose order varies) and
//                       divides by the squared-window sum; trims the centre
//                       padding and pads / truncates to the requested length.
#include <algorithm>

#include "fft_core.hpp"
#include "msst_common.hpp"

namespace msst {
namespace {

using fft::cf;
constexpr int kFftThreads = 256;

// Forward M-point FFT of `a` using `b` as the second buffer; returns the
// buffer that holds the result.  Every thread of the block takes part.
__device__ cf* fft_lds(cf* a, cf* b, int M) {
    cf* src = a;
    cf* dst = b;
    int Ns = 1;
    for (; 4 * Ns <= M; Ns *= 4) {
        for (int j = threadIdx.x; j < (M >> 2); j += blockDim.x) fft::radix4(src, dst, j, Ns, M);
        __syncthreads();
        cf* t = src;
        src = dst;
        dst = t;
    }
    if (Ns < M) {
        for (int j = threadIdx.x; j < (M >> 1); j += blockDim.x) fft::radix2(src, dst, j, Ns, M);
        __syncthreads();
        cf* t = src;
        src = dst;
        dst = t;
    }
    return src;
}

__global__ __launch_bounds__(kFftThreads) void stft_kernel(const float* __restrict__ sig, int L,
                                                           int T, int hop, int n_fft, int pad,
                                                           const float* __restrict__ window,
                                                           float scale, float2* __restrict__ out) {
    extern __shared__ cf lds[];
    const int M = n_fft >> 1, F = M + 1;
    const int t = blockIdx.x, bc = blockIdx.y;
    cf* a = lds;
    cf* b = lds + M;
    const float* s = sig + (int64_t)bc * L;
    const int base = t * hop - pad;
    for (int n = threadIdx.x; n < M; n += blockDim.x) {
        float v[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int i = 2 * n + e;
            int p = base + i;
            if (p < 0) p = -p;                  // reflect (edge sample not repeated)
            if (p >= L) p = 2 * (L - 1) - p;
            v[e] = s[p] * window[i];
        }
        a[n] = cf{v[0], v[1]};
    }
    __syncthreads();
    const cf* Z = fft_lds(a, b, M);
    float2* o = out + (int64_t)bc * F * T + t;
    for (int k = threadIdx.x; k <= (M >> 1); k += blockDim.x) {
        cf xk, xmk;
        fft::r2c_unpack(Z, k, M, xk, xmk);
        o[(int64_t)k * T] = float2{xk.x * scale, xk.y * scale};
        if (M - k != k) o[(int64_t)(M - k) * T] = float2{xmk.x * scale, xmk.y * scale};
    }
}

__global__ __launch_bounds__(kFftThreads) void istft_frame_kernel(
    const float2* __restrict__ spec, int T, int n_fft, const float* __restrict__ window,
    float scale, float* __restrict__ frames) {
    extern __shared__ cf lds[];
    const int M = n_fft >> 1, F = M + 1;
    const int t = blockIdx.x, bc = blockIdx.y;
    cf* a = lds;          // M entries
    cf* b = lds + M;      // M + 1 entries (the bins, then the FFT's second buffer)
    const float2* sp = spec + (int64_t)bc * F * T + t;
    for (int k = threadIdx.x; k < F; k += blockDim.x) {
        const float2 v = sp[(int64_t)k * T];
        b[k] = cf{v.x * scale, v.y * scale};
    }
    __syncthreads();
    // Z[k] from the bins (imaginary parts of bins 0 and M are ignored, as a
    // Hermitian C2R transform does); store conj(Z) so a forward FFT gives
    // conj(M z).
    for (int k = threadIdx.x; k <= (M >> 1); k += blockDim.x) {
        cf zk, zmk;
        fft::c2r_pack(b[k], b[M - k], k, M, zk, zmk);
        a[k] = fft::cconj(zk);
        if (k != 0 && M - k != k) a[M - k] = fft::cconj(zmk);
    }
    __syncthreads();
    const cf* r = fft_lds(a, b, M);
    const float inv = 1.0f / (float)M;
    float* fr = frames + ((int64_t)bc * T + t) * n_fft;
    for (int n = threadIdx.x; n < M; n += blockDim.x) {
        const cf v = r[n];  // conj(M z[n])
        fr[2 * n] = v.x * inv * window[2 * n];
        fr[2 * n + 1] = -v.y * inv * window[2 * n + 1];
    }
}

__global__ __launch_bounds__(256) void istft_ola_kernel(const float* __restrict__ frames, int T,
                                                        int n_fft, int hop, int pad,
                                                        int valid, int out_len,
                                                        const float* __restrict__ window,
                                                        float* __restrict__ out) {
    const int o = blockIdx.x * blockDim.x + threadIdx.x;
    const int bc = blockIdx.y;
    if (o >= out_len) return;
    float v = 0.0f;
    if (o < valid) {
        const int pos = o + pad;
        const int t_hi = min(T - 1, pos / hop);
        const int t_lo = pos >= n_fft ? (pos - n_fft) / hop + 1 : 0;
        float acc = 0.0f, ws = 0.0f;
        const float* fb = frames + (int64_t)bc * T * n_fft;
        for (int t = t_lo; t <= t_hi; ++t) {
            const int n = pos - t * hop;
            const float w = window[n];
            acc += fb[(int64_t)t * n_fft + n];
            ws += w * w;
        }
        v = ws > 1e-8f ? acc / ws : acc;
    }
    out[(int64_t)bc * out_len + o] = v;
}

__global__ __launch_bounds__(256) void hann_kernel(float* out, int size) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < size) out[i] = size == 1 ? 1.0f : 0.5f * (1.0f - cospif(2.0f * (float)i / (float)size));
}

// Power-of-two sizes whose two LDS buffers ((n_fft + 2) complex values) fit
// the 64 KB a launch gets without raising the dynamic-LDS limit.
int fft_ok(int n_fft) {
    return n_fft >= 16 && n_fft <= 4096 && (n_fft & (n_fft - 1)) == 0;
}

}  // namespace
}  // namespace msst

using namespace msst;

extern "C" int64_t msst_stft_frames(int64_t length, int n_fft, int hop, int center) {
    if (!fft_ok(n_fft) || hop < 1 || length < 1) return -1;
    const int64_t padded = length + (center ? n_fft : 0);
    if (padded < n_fft || (center && length <= n_fft / 2)) return -1;
    return (padded - n_fft) / hop + 1;
}

extern "C" int msst_stft(const float* signal, int64_t batch, int64_t length, int n_fft, int hop,
                         const float* window, int center, int normalized, float* out,
                         void* stream) {
    MSST_REQUIRE(signal && window && out, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(fft_ok(n_fft), MSST_ERR_UNSUPPORTED, "n_fft must be a power of two in [16, 4096]");
    MSST_REQUIRE(hop >= 1 && batch >= 0 && batch < 65536 && length < (1 << 30),
                 MSST_ERR_INVALID_ARG, "bad hop / batch / length");
    const int64_t T = msst_stft_frames(length, n_fft, hop, center);
    MSST_REQUIRE(T >= 1, MSST_ERR_INVALID_ARG,
                 "signal too short (centre reflect padding needs length > n_fft / 2)");
    MSST_REQUIRE(aligned(out, 8), MSST_ERR_ALIGNMENT, "out must be 8-byte aligned");
    if (batch == 0) return MSST_OK;
    const float scale = normalized ? 1.0f / sqrtf((float)n_fft) : 1.0f;
    const size_t lds = (size_t)(n_fft + 2) * sizeof(cf);
    hipLaunchKernelGGL(stft_kernel, dim3((unsigned)T, (unsigned)batch), dim3(kFftThreads), lds,
                       as_stream(stream), signal, (int)length, (int)T, hop, n_fft,
                       center ? n_fft / 2 : 0, window, scale, reinterpret_cast<float2*>(out));
    return check_launch("stft_kernel");
}

extern "C" int64_t msst_istft_length(int64_t frames, int n_fft, int hop, int64_t length,
                                     int center) {
    if (!fft_ok(n_fft) || hop < 1 || frames < 1) return -1;
    if (length > 0) return length;
    return (int64_t)n_fft + (frames - 1) * hop - (center ? n_fft : 0);
}

extern "C" int64_t msst_istft_workspace(int64_t batch, int64_t frames, int n_fft) {
    if (batch < 0 || frames < 0 || n_fft < 1) return -1;
    return batch * frames * n_fft * 4;
}

extern "C" int msst_istft(const float* spec, int64_t batch, int64_t frames, int n_fft, int hop,
                          const float* window, int64_t length, int center, int normalized,
                          float* out, void* workspace, int64_t ws_bytes, void* stream) {
    MSST_REQUIRE(spec && window && out && workspace, MSST_ERR_INVALID_ARG, "null pointer");
    MSST_REQUIRE(fft_ok(n_fft), MSST_ERR_UNSUPPORTED, "n_fft must be a power of two in [16, 4096]");
    MSST_REQUIRE(hop >= 1 && hop <= n_fft && batch >= 0 && batch < 65536 && frames >= 1 &&
                     frames < (1 << 24),
                 MSST_ERR_INVALID_ARG, "bad hop / batch / frames");
    const int64_t out_len = msst_istft_length(frames, n_fft, hop, length, center);
    MSST_REQUIRE(out_len >= 1 && out_len < (1 << 30), MSST_ERR_INVALID_ARG, "bad output length");
    MSST_REQUIRE(ws_bytes >= msst_istft_workspace(batch, frames, n_fft), MSST_ERR_WORKSPACE,
                 "workspace too small");
    MSST_REQUIRE(aligned(spec, 8) && aligned(workspace, 16), MSST_ERR_ALIGNMENT,
                 "spec 8-byte, workspace 16-byte aligned");
    if (batch == 0) return MSST_OK;
    hipStream_t s = as_stream(stream);
    const float scale = normalized ? sqrtf((float)n_fft) : 1.0f;
    float* fr = reinterpret_cast<float*>(workspace);
    const size_t lds = (size_t)(n_fft + 2) * sizeof(cf);
    hipLaunchKernelGGL(istft_frame_kernel, dim3((unsigned)frames, (unsigned)batch),
                       dim3(kFftThreads), lds, s, reinterpret_cast<const float2*>(spec),
                       (int)frames, n_fft, window, scale, fr);
    int rc = check_launch("istft_frame_kernel");
    if (rc != MSST_OK) return rc;
    const int pad = center ? n_fft / 2 : 0;
    const int64_t full = (int64_t)n_fft + (frames - 1) * hop;
    const int valid = (int)std::min<int64_t>(out_len, full - 2 * pad);
    hipLaunchKernelGGL(istft_ola_kernel,
                       dim3((unsigned)((out_len + 255) / 256), (unsigned)batch), dim3(256), 0, s,
                       fr, (int)frames, n_fft, hop, pad, valid, (int)out_len, window, out);
    return check_launch("istft_ola_kernel");
}

extern "C" int msst_hann_window(float* out, int size, void* stream) {
    MSST_REQUIRE(out && size >= 1, MSST_ERR_INVALID_ARG, "bad window");
    hipLaunchKernelGGL(hann_kernel, dim3((unsigned)((size + 255) / 256)), dim3(256), 0,
                       as_stream(stream), out, size);
    return check_launch("hann_kernel");
}
