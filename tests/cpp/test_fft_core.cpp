// CPU check of the FFT arithmetic the STFT kernels use (csrc/fft_core.hpp):
// the Stockham passes run sequentially in the order the kernel's barriers
// impose, and the real-transform pack / unpack, against a float64 DFT.
// Exercises the same index and twiddle code the GPU runs, so an indexing
// mistake shows here before any launch.
#include <cmath>
#include <complex>
#include <cstdio>
#include <random>
#include <vector>

#include "fft_core.hpp"

using msst::fft::cf;
typedef std::complex<double> cd;

static int g_fail = 0;

static cf* fft_host(cf* a, cf* b, int M) {  // mirrors fft_lds in stft.hip
    cf* src = a;
    cf* dst = b;
    int Ns = 1;
    for (; 4 * Ns <= M; Ns *= 4) {
        for (int j = 0; j < (M >> 2); ++j) msst::fft::radix4(src, dst, j, Ns, M);
        std::swap(src, dst);
    }
    if (Ns < M) {
        for (int j = 0; j < (M >> 1); ++j) msst::fft::radix2(src, dst, j, Ns, M);
        std::swap(src, dst);
    }
    return src;
}

static void check(const char* what, int N, double err, double tol) {
    std::printf("%-28s N=%5d  max rel err %.2e\n", what, N, err);
    if (!(err <= tol)) {
        std::printf("FAIL: %s N=%d (tol %.1e)\n", what, N, tol);
        ++g_fail;
    }
}

int main() {
    std::mt19937 rng(1);
    std::normal_distribution<double> nd;
    for (int N = 16; N <= 8192; N *= 2) {
        const int M = N / 2;
        std::vector<double> x(N);
        for (auto& v : x) v = nd(rng);
        // float64 DFT of the real signal, bins 0..M
        std::vector<cd> X(M + 1);
        double xmax = 0;
        for (int k = 0; k <= M; ++k) {
            cd acc = 0;
            for (int n = 0; n < N; ++n) acc += x[n] * std::polar(1.0, -2.0 * M_PI * k * n / N);
            X[k] = acc;
            xmax = std::max(xmax, std::abs(acc));
        }
        // forward: pack, FFT, unpack
        std::vector<cf> a(M), b(M);
        for (int n = 0; n < M; ++n) a[n] = cf{(float)x[2 * n], (float)x[2 * n + 1]};
        const cf* Z = fft_host(a.data(), b.data(), M);
        std::vector<cf> Y(M + 1);
        for (int k = 0; k <= M / 2; ++k) {
            cf xk, xmk;
            msst::fft::r2c_unpack(Z, k, M, xk, xmk);
            Y[k] = xk;
            if (M - k != k) Y[M - k] = xmk;
        }
        double e = 0;
        for (int k = 0; k <= M; ++k) e = std::max(e, std::abs(cd(Y[k].x, Y[k].y) - X[k]));
        check("r2c (pack + FFT + unpack)", N, e / xmax, 4e-6);
        // inverse: pack conj(Z), FFT, conj / M -> x
        std::vector<cf> bins(M + 1);
        for (int k = 0; k <= M; ++k) bins[k] = cf{(float)X[k].real(), (float)X[k].imag()};
        bins[0].y = 123.0f;  // ignored (Hermitian C2R)
        bins[M].y = -7.0f;
        for (int k = 0; k <= M / 2; ++k) {
            cf zk, zmk;
            msst::fft::c2r_pack(bins[k], bins[M - k], k, M, zk, zmk);
            a[k] = msst::fft::cconj(zk);
            if (k != 0 && M - k != k) a[M - k] = msst::fft::cconj(zmk);
        }
        const cf* r = fft_host(a.data(), b.data(), M);
        double ei = 0, amax = 0;
        for (int n = 0; n < M; ++n) {
            ei = std::max(ei, std::fabs(r[n].x / M - x[2 * n]));
            ei = std::max(ei, std::fabs(-r[n].y / M - x[2 * n + 1]));
        }
        for (double v : x) amax = std::max(amax, std::fabs(v));
        check("c2r (pack + FFT + unpack)", N, ei / amax, 4e-6);
    }
    std::printf("%s\n", g_fail ? "FAILED" : "OK");
    return g_fail ? 1 : 0;
}
