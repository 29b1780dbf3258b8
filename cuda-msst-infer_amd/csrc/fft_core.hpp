// fft_core.hpp — the arithmetic of the STFT kernels (stft.hip), written as
// host+device functions so the same code runs in the kernels and in a CPU
// check of its indexing.
//
// Complex FFT of M = 2^m points: Stockham auto-sort (Govindaraju et al.,
// "High Performance Discrete Fourier Transforms on Graphics Processors",
// SC 2008): pass p reads sub-transform outputs of size Ns from `src`,
// multiplies by the twiddles exp(-2 pi i (j mod Ns) r / (R Ns)), does an R-point
// DFT and writes to position (j / Ns) * Ns * R + j mod Ns + r * Ns of `dst`.
// Radix-4 passes while 4 Ns <= M, then one radix-2 pass when log2 M is odd.
//
// Real transform of N = 2M points through the M-point complex one (the
// standard packing z[n] = x[2n] + i x[2n+1]):
//   X[k] = Xe[k] + W^k Xo[k],   Xe[k] = (Z[k] + conj Z[M-k]) / 2,
//   Xo[k] = (Z[k] - conj Z[M-k]) / (2i),   W = exp(-2 pi i / N),
// and back: Xe[k] = (X[k] + conj X[M-k]) / 2, Xo[k] = (X[k] - conj X[M-k]) W^-k / 2,
// Z[k] = Xe[k] + i Xo[k].
#pragma once

#include <hip/hip_runtime.h>

namespace msst {
namespace fft {

struct cf {
    float x, y;
};

__host__ __device__ inline cf cadd(cf a, cf b) { return {a.x + b.x, a.y + b.y}; }
__host__ __device__ inline cf csub(cf a, cf b) { return {a.x - b.x, a.y - b.y}; }
__host__ __device__ inline cf cmul(cf a, cf b) {
    return {a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x};
}
__host__ __device__ inline cf cconj(cf a) { return {a.x, -a.y}; }
__host__ __device__ inline cf cscale(cf a, float s) { return {a.x * s, a.y * s}; }
__host__ __device__ inline cf mul_mi(cf a) { return {a.y, -a.x}; }  // a * (-i)
__host__ __device__ inline cf mul_pi(cf a) { return {-a.y, a.x}; }  // a * (+i)

// exp(i pi t) (t in half-turns).
__host__ __device__ inline cf expi_pi(float t) {
    float s, c;
#ifdef __HIP_DEVICE_COMPILE__
    sincospif(t, &s, &c);
#else
    s = (float)sin(3.14159265358979323846 * (double)t);
    c = (float)cos(3.14159265358979323846 * (double)t);
#endif
    return {c, s};
}

// Butterfly j of a radix-4 pass (j < M / 4).
__host__ __device__ inline void radix4(const cf* src, cf* dst, int j, int Ns, int M) {
    const int q = M >> 2;
    const int k = j & (Ns - 1);
    cf v0 = src[j], v1 = src[j + q], v2 = src[j + 2 * q], v3 = src[j + 3 * q];
    if (Ns > 1) {
        const float t = -2.0f * (float)k / (float)(4 * Ns);  // half-turns
        v1 = cmul(v1, expi_pi(t));
        v2 = cmul(v2, expi_pi(2.0f * t));
        v3 = cmul(v3, expi_pi(3.0f * t));
    }
    const cf a0 = cadd(v0, v2), a1 = csub(v0, v2), a2 = cadd(v1, v3), a3 = csub(v1, v3);
    const int d = ((j - k) << 2) + k;
    dst[d] = cadd(a0, a2);
    dst[d + Ns] = cadd(a1, mul_mi(a3));
    dst[d + 2 * Ns] = csub(a0, a2);
    dst[d + 3 * Ns] = csub(a1, mul_mi(a3));
}

// Butterfly j of the final radix-2 pass (j < M / 2, 2 Ns == M).
__host__ __device__ inline void radix2(const cf* src, cf* dst, int j, int Ns, int M) {
    const int k = j & (Ns - 1);
    cf v0 = src[j], v1 = src[j + (M >> 1)];
    v1 = cmul(v1, expi_pi(-2.0f * (float)k / (float)(2 * Ns)));
    const int d = ((j - k) << 1) + k;
    dst[d] = cadd(v0, v1);
    dst[d + Ns] = csub(v0, v1);
}

// Real-transform unpack for the bin pair (k, M - k), 0 <= k <= M / 2; Z has
// M entries; writes X[k] and X[M - k] (for k = 0: X[0] and X[M]).
__host__ __device__ inline void r2c_unpack(const cf* Z, int k, int M, cf& xk, cf& xmk) {
    if (k == 0) {
        xk = {Z[0].x + Z[0].y, 0.0f};
        xmk = {Z[0].x - Z[0].y, 0.0f};
        return;
    }
    const cf a = Z[k], b = cconj(Z[M - k]);
    const cf xe = cscale(cadd(a, b), 0.5f);
    const cf xo = cscale(mul_mi(csub(a, b)), 0.5f);  // (a - b) / (2i)
    const cf w = expi_pi(-(float)k / (float)M);      // W^k, N = 2M
    xk = cadd(xe, cmul(w, xo));
    // X[M - k] = conj(Xe[k]) - W^-k conj(Xo[k]) = conj(Xe[k] - W^k Xo[k])
    xmk = cconj(csub(xe, cmul(w, xo)));
}

// Inverse pack for the bin pair (k, M - k), 0 < k <= M / 2: Z[k], Z[M - k]
// from X[k], X[M - k].  k = 0 uses X[0] and X[M] (imaginary parts ignored).
__host__ __device__ inline void c2r_pack(cf xk, cf xmk, int k, int M, cf& zk, cf& zmk) {
    if (k == 0) {
        const float e = 0.5f * (xk.x + xmk.x), o = 0.5f * (xk.x - xmk.x);
        zk = {e, o};  // Xe[0] + i Xo[0]
        zmk = zk;
        return;
    }
    const cf w = expi_pi(-(float)k / (float)M);  // W^k
    const cf winv = cconj(w);
    {
        const cf b = cconj(xmk);
        const cf xe = cscale(cadd(xk, b), 0.5f);
        const cf xo = cscale(cmul(csub(xk, b), winv), 0.5f);
        zk = cadd(xe, mul_pi(xo));
    }
    {
        // the same for index M - k: W^(M-k) = -W^-k, so W^-(M-k) = -W^k.
        const cf b = cconj(xk);
        const cf xe = cscale(cadd(xmk, b), 0.5f);
        const cf xo = cscale(cmul(csub(xmk, b), cscale(w, -1.0f)), 0.5f);
        zmk = cadd(xe, mul_pi(xo));
    }
}

}  // namespace fft
}  // namespace msst
