// test_host_ops.cpp — the cudasep::ops / Tensor C++ surface on the GPU,
// checked against the CPU oracle (oracle/msst_oracle.h) on the same seeded
// inputs, plus the reference's dtype rules and error behaviour.
//
// Tolerances (normwise max|y - r| / max|r|): 1e-4 for fp32 weights, 2e-2
// for fp16 outputs; fp32 outputs of fp16 GEMMs use 1e-3 (the oracle is fed
// the fp16-rounded operands, so only accumulation order differs).
// Exit status 0 when every check passes.
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "msst_oracle.h"
#include "ops.h"

using cudasep::DType;
using cudasep::Tensor;
namespace ops = cudasep::ops;

static int g_checks = 0, g_fail = 0;

static void expect(bool ok, const std::string& what) {
    ++g_checks;
    if (!ok) {
        ++g_fail;
        std::printf("FAIL: %s\n", what.c_str());
    }
}

static std::vector<float> randn(size_t n, float sd, uint64_t seed, float mean = 0.0f) {
    std::mt19937_64 g(seed);
    std::normal_distribution<float> d(mean, sd);
    std::vector<float> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

static std::vector<float> round16(std::vector<float> v) {
    for (auto& x : v) x = __half2float(__float2half(x));
    return v;
}

static Tensor dev(const std::vector<float>& v, std::vector<int64_t> shape, DType dt) {
    Tensor t = Tensor::from_cpu_f32(v.data(), shape);
    return t.to_dtype(dt);
}

static double rel_err(const std::vector<float>& y, const std::vector<float>& r) {
    double num = 0, den = 0;
    for (size_t i = 0; i < r.size(); ++i) {
        num = std::fmax(num, std::fabs((double)y[i] - r[i]));
        den = std::fmax(den, std::fabs((double)r[i]));
    }
    if (!std::isfinite(num)) return INFINITY;
    return den > 0 ? num / den : num;
}

static void check_close(const std::string& name, const Tensor& y, const std::vector<float>& r,
                        double tol) {
    const std::vector<float> h = y.to_cpu_f32();
    const double e = h.size() == r.size() ? rel_err(h, r) : INFINITY;
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s: rel err %.3e (tol %.1e)", name.c_str(), e, tol);
    std::printf("%s\n", buf);
    expect(e <= tol, buf);
}

template <typename F>
static void expect_throw(const std::string& name, F f) {
    bool threw = false;
    try {
        f();
    } catch (const std::exception& ex) {
        threw = true;
        std::printf("%s: threw \"%s\"\n", name.c_str(), ex.what());
    }
    expect(threw, name + " should throw");
}

static void test_linear() {
    const int64_t M = 300, K = 512, N = 384;
    auto x = round16(randn(M * K, 1.0f, 1));
    auto w = round16(randn(N * K, 0.02f, 2));
    auto b = randn(N, 0.02f, 3);
    std::vector<float> r(M * N), rg(M * N), rs(M * N), rsi(M * N), rn(M * N);
    orc_linear(x.data(), w.data(), b.data(), nullptr, r.data(), M, K, N, ORC_ACT_NONE);
    orc_linear(x.data(), w.data(), b.data(), nullptr, rg.data(), M, K, N, ORC_ACT_GELU);
    orc_linear(x.data(), w.data(), b.data(), nullptr, rs.data(), M, K, N, ORC_ACT_SIGMOID);
    orc_linear(x.data(), w.data(), b.data(), nullptr, rsi.data(), M, K, N, ORC_ACT_SILU);
    orc_linear(x.data(), w.data(), nullptr, nullptr, rn.data(), M, K, N, ORC_ACT_NONE);

    Tensor xf = dev(x, {3, 100, K}, DType::Float32), xh = xf.to_f16();
    Tensor wh = dev(w, {N, K}, DType::Float16), wf = wh.to_f32();
    Tensor bf = dev(b, {N}, DType::Float32), bh = bf.to_f16();

    // fp16 W: linear / linear_no_bias return fp32 whatever x is.
    Tensor y = ops::linear(xf, wh, bf);
    expect(y.dtype() == DType::Float32 && y.shape() == std::vector<int64_t>({3, 100, N}),
           "linear(f32 x, f16 W) -> fp32 [3,100,N], got " + y.shape_str());
    check_close("linear f16 W, f32 x", y, r, 1e-3);
    Tensor y2 = ops::linear(xh, wh, bf);
    expect(y2.dtype() == DType::Float32, "linear(f16 x, f16 W) -> fp32");
    check_close("linear f16 W, f16 x", y2, r, 1e-3);
    check_close("linear f16 W, f16 bias promoted", ops::linear(xf, wh, bh), r, 1e-3);
    Tensor yn = ops::linear_no_bias(xf, wh);
    expect(yn.dtype() == DType::Float32, "linear_no_bias(f16 W) -> fp32");
    check_close("linear_no_bias f16 W", yn, rn, 1e-3);

    // fp32 W: the output follows x.
    Tensor y3 = ops::linear(xf, wf, bf);
    expect(y3.dtype() == DType::Float32, "linear(f32 x, f32 W) -> fp32");
    check_close("linear f32 W", y3, r, 1e-4);
    Tensor y4 = ops::linear(xh, wf, bf);
    expect(y4.dtype() == DType::Float16, "linear(f16 x, f32 W) -> fp16");
    check_close("linear f32 W, f16 x", y4, r, 2e-2);

    // Fused activations: fp16 out iff x is fp16.
    Tensor g1 = ops::linear_gelu(xf, wh, bf);
    expect(g1.dtype() == DType::Float32, "linear_gelu(f32 x) -> fp32");
    check_close("linear_gelu f16 W, f32 x", g1, rg, 1e-3);
    Tensor g2 = ops::linear_gelu(xh, wh, bf);
    expect(g2.dtype() == DType::Float16, "linear_gelu(f16 x) -> fp16");
    check_close("linear_gelu f16 W, f16 x", g2, rg, 2e-2);
    check_close("linear_sigmoid f16 W", ops::linear_sigmoid(xf, wh, bf), rs, 1e-3);
    check_close("linear_silu f16 W", ops::linear_silu(xf, wh, bf), rsi, 1e-3);
    check_close("linear_gelu f32 W", ops::linear_gelu(xf, wf, bf), rg, 1e-4);

    expect_throw("linear with mismatched in_features",
                 [&] { ops::linear(dev(x, {M * K / 256, 256}, DType::Float32), wh, bf); });
    expect_throw("linear with a short bias",
                 [&] { ops::linear(xf, wh, dev(b, {N - 1}, DType::Float32)); });
}

static void test_rms_norm() {
    const int64_t rows = 777, D = 512;
    auto x = randn(rows * D, 1.0f, 4);
    auto g = randn(D, 0.02f, 5, 1.0f);
    std::vector<float> r(rows * D);
    orc_rms_norm(x.data(), g.data(), std::sqrt((float)D), r.data(), rows, D);
    Tensor xf = dev(x, {7, 111, D}, DType::Float32);
    Tensor gf = dev(g, {D}, DType::Float32);
    Tensor y = ops::rms_norm(xf, gf, std::sqrt((float)D));
    expect(y.dtype() == DType::Float32 && y.shape() == xf.shape(), "rms_norm keeps f32 and shape");
    check_close("rms_norm f32", y, r, 1e-4);
    auto xr = round16(x);
    std::vector<float> r16(rows * D);
    orc_rms_norm(xr.data(), g.data(), std::sqrt((float)D), r16.data(), rows, D);
    Tensor yh = ops::rms_norm(xf.to_f16(), gf.to_f16(), std::sqrt((float)D));
    expect(yh.dtype() == DType::Float16, "rms_norm keeps f16");
    check_close("rms_norm f16 (f16 gamma promoted)", yh, r16, 2e-3);
    expect_throw("rms_norm with a wrong gamma",
                 [&] { ops::rms_norm(xf, dev(g, {D / 2}, DType::Float32), 1.0f); });
}

static void test_rope_attention() {
    const int64_t B = 2, H = 8, N = 801, Nk = 801, D = 64;
    std::vector<float> c(N * D / 2), s(N * D / 2);
    orc_rope_table((int)N, (int)D, c.data(), s.data());
    Tensor ct = dev(c, {N, D / 2}, DType::Float32), st = dev(s, {N, D / 2}, DType::Float32);
    for (DType dt : {DType::Float32, DType::Float16}) {
        const bool h = dt == DType::Float16;
        auto q = randn(B * H * N * D, 1.0f, 6), k = randn(B * H * Nk * D, 1.0f, 7),
             v = randn(B * H * Nk * D, 1.0f, 8);
        if (h) q = round16(q), k = round16(k), v = round16(v);
        Tensor qd = dev(q, {B, H, N, D}, dt), kd = dev(k, {B, H, Nk, D}, dt),
               vd = dev(v, {B, H, Nk, D}, dt);
        // RoPE in place.
        std::vector<float> qr = q, kr = k;
        orc_rope_apply(qr.data(), kr.data(), c.data(), s.data(), B, H, N, D);
        ops::apply_rotary_emb(qd, kd, ct, st);
        expect(qd.dtype() == dt, "apply_rotary_emb keeps dtype");
        check_close(std::string("apply_rotary_emb q ") + (h ? "f16" : "f32"), qd, qr, h ? 2e-3 : 1e-4);
        check_close(std::string("apply_rotary_emb k ") + (h ? "f16" : "f32"), kd, kr, h ? 2e-3 : 1e-4);
        // Attention on the rotated q, k (the device copies are what the
        // oracle gets, rounded as stored).
        auto qh = qd.to_cpu_f32(), kh = kd.to_cpu_f32();
        std::vector<float> r(B * H * N * D);
        orc_attention(qh.data(), kh.data(), v.data(), r.data(), B, H, N, Nk, D,
                      1.0f / std::sqrt((float)D));
        Tensor o = ops::scaled_dot_product_attention(qd, kd, vd);
        expect(o.dtype() == dt && o.shape() == qd.shape(), "sdpa keeps dtype and shape");
        check_close(std::string("scaled_dot_product_attention ") + (h ? "f16" : "f32"), o, r,
                    h ? 2e-2 : 1e-4);
    }
    // Head dims other than 64 (the reference takes any D): a ragged case
    // through the generic kernel, and D > 256 refused.
    for (DType dt : {DType::Float32, DType::Float16}) {
        const bool h = dt == DType::Float16;
        const int64_t b = 1, hh = 2, n = 70, nk = 45, d = 40;
        auto q = randn(b * hh * n * d, 1.0f, 16), k = randn(b * hh * nk * d, 1.0f, 17),
             v = randn(b * hh * nk * d, 1.0f, 18);
        if (h) q = round16(q), k = round16(k), v = round16(v);
        std::vector<float> r(b * hh * n * d);
        orc_attention(q.data(), k.data(), v.data(), r.data(), b, hh, n, nk, d,
                      1.0f / std::sqrt((float)d));
        Tensor o = ops::scaled_dot_product_attention(dev(q, {b, hh, n, d}, dt),
                                                     dev(k, {b, hh, nk, d}, dt),
                                                     dev(v, {b, hh, nk, d}, dt));
        check_close(std::string("scaled_dot_product_attention D=40 ") + (h ? "f16" : "f32"), o, r,
                    h ? 2e-2 : 1e-4);
    }
    expect_throw("sdpa with head dim 300", [&] {
        Tensor q = Tensor::zeros({1, 1, 4, 300});
        ops::scaled_dot_product_attention(q, q, q);
    });
    expect_throw("apply_rotary_emb on 3-D q", [&] {
        Tensor q = Tensor::zeros({1, 4, 64});
        ops::apply_rotary_emb(q, q, ct, st);
    });
}

static void test_stack() {
    const int64_t B = 1, T = 40, F = 6, dim = 128, H = 2, Dh = 64, ff = 512, depth = 2;
    std::vector<std::vector<float>> store;
    std::vector<orc_layer_weights> ow(2 * depth);
    std::vector<ops::RoformerLayer> lw(2 * depth);
    uint64_t seed = 100;
    auto mat = [&](int64_t r, int64_t cols) {
        store.push_back(round16(randn(r * cols, 0.02f, seed++)));
        return &store.back();
    };
    auto gam = [&]() {
        store.push_back(randn(dim, 0.02f, seed++, 1.0f));
        return &store.back();
    };
    store.reserve(64);
    for (int64_t i = 0; i < 2 * depth; ++i) {
        auto* ag = gam(); auto* wq = mat(3 * H * Dh, dim); auto* wg = mat(H, dim);
        auto* bg = mat(H, 1); auto* wo = mat(dim, H * Dh); auto* fg = gam();
        auto* w1 = mat(ff, dim); auto* b1 = mat(ff, 1); auto* w2 = mat(dim, ff); auto* b2 = mat(dim, 1);
        ow[i] = orc_layer_weights{ag->data(), wq->data(), wg->data(), bg->data(), wo->data(),
                                  fg->data(), w1->data(), b1->data(), w2->data(), b2->data(),
                                  nullptr};
        lw[i].attn_gamma = dev(*ag, {dim}, DType::Float32);
        lw[i].w_qkv = dev(*wq, {3 * H * Dh, dim}, DType::Float16);
        lw[i].w_gate = dev(*wg, {H, dim}, DType::Float16);
        lw[i].b_gate = dev(*bg, {H}, DType::Float32);
        lw[i].w_out = dev(*wo, {dim, H * Dh}, DType::Float16);
        lw[i].ff_gamma = dev(*fg, {dim}, DType::Float32);
        lw[i].w_ff1 = dev(*w1, {ff, dim}, DType::Float16);
        lw[i].b_ff1 = dev(*b1, {ff}, DType::Float32);
        lw[i].w_ff2 = dev(*w2, {dim, ff}, DType::Float16);
        lw[i].b_ff2 = dev(*b2, {dim}, DType::Float32);
    }
    auto* fgam = gam();
    auto x = randn(B * T * F * dim, 1.0f, 99);
    std::vector<float> r = x;
    orc_roformer_stack(r.data(), B, T, F, dim, H, Dh, ff, depth, ow.data(), fgam->data());
    Tensor xd = dev(x, {B, T, F, dim}, DType::Float32);
    ops::roformer_stack(xd, lw, (int)H, (int)Dh, dev(*fgam, {dim}, DType::Float32));
    check_close("roformer_stack fp16 [1,40,6,128] depth 2", xd, r, 2e-2);
}

static void test_tensor() {
    Tensor t = Tensor::zeros({2, 3, 4});
    expect(t.numel() == 24 && t.size(-1) == 4 && t.ndim() == 3, "Tensor shape queries");
    expect(t.reshape({-1, 4}).shape() == std::vector<int64_t>({6, 4}), "reshape infers -1");
    expect_throw("Tensor::size out of range", [&] { (void)t.size(3); });
    expect_throw("reshape to a wrong count", [&] { (void)t.reshape({5, 5}); });
    expect_throw("add_ with a dtype mismatch", [&] { t.add_(t.to_f16()); });
    auto v = randn(24, 1.0f, 11);
    Tensor a = dev(v, {2, 3, 4}, DType::Float32);
    Tensor s = a + a;
    auto h = s.to_cpu_f32();
    bool ok = true;
    for (size_t i = 0; i < v.size(); ++i) ok = ok && h[i] == 2 * v[i];
    expect(ok, "operator+ is exact");
}

static void test_bands() {
    // tanh_act / glu (ops.h:36, :116)
    const int64_t R = 37, H2 = 26;
    auto x = randn(R * 2 * H2, 2.0f, 41);
    std::vector<float> rt(x.size()), rg(R * H2);
    orc_activation(x.data(), rt.data(), (int64_t)x.size(), ORC_ACT_TANH);
    orc_glu(x.data(), rg.data(), R, H2);
    Tensor xd = dev(x, {R, 2 * H2}, DType::Float32);
    check_close("tanh_act f32", ops::tanh_act(xd), rt, 1e-6);
    Tensor g = ops::glu(xd, -1);
    expect(g.shape() == std::vector<int64_t>({R, H2}), "glu halves the last dim");
    check_close("glu f32", g, rg, 1e-6);
    expect_throw("glu on an odd last dim", [&] { ops::glu(xd.reshape({-1, 13}), -1); });

    // BandPlan: 5 bands of a stereo split, dim 64, MLP of 2 linears (hidden 128).
    const std::vector<int> dims = {4, 8, 16, 48, 516};
    const int nb = (int)dims.size(), dim = 64, hid = 128, L = 2;
    int ftot = 0;
    for (int d : dims) ftot += d;
    const int64_t B = 2, T = 31, rows = B * T;
    ops::BandSplitWeights sw;
    ops::MaskEstimatorWeights mw;
    std::vector<float> gcat, wcat, bcat, mwcat, mbcat;
    for (int b = 0; b < nb; ++b) {
        auto gam = randn(dims[b], 0.02f, 100 + b, 1.0f);
        auto w = round16(randn((size_t)dim * dims[b], 1.0f / std::sqrt((float)dims[b]), 200 + b));
        auto bb = randn(dim, 0.02f, 300 + b);
        sw.gamma.push_back(dev(gam, {dims[b]}, DType::Float32));
        sw.w.push_back(dev(w, {dim, dims[b]}, DType::Float16));
        sw.b.push_back(dev(bb, {dim}, DType::Float32));
        gcat.insert(gcat.end(), gam.begin(), gam.end());
        wcat.insert(wcat.end(), w.begin(), w.end());
        bcat.insert(bcat.end(), bb.begin(), bb.end());
        std::vector<Tensor> wl, bl;
        int K = dim;
        for (int l = 0; l < L; ++l) {
            const int N = l == L - 1 ? 2 * dims[b] : hid;
            auto ww = round16(randn((size_t)N * K, 1.0f / std::sqrt((float)K), 400 + 10 * b + l));
            auto wb = randn(N, 0.02f, 500 + 10 * b + l);
            wl.push_back(dev(ww, {N, K}, DType::Float16));
            bl.push_back(dev(wb, {N}, DType::Float16));  // fp16 bias is promoted
            mwcat.insert(mwcat.end(), ww.begin(), ww.end());
            auto wb16 = round16(wb);
            mbcat.insert(mbcat.end(), wb16.begin(), wb16.end());
            K = N;
        }
        mw.w.push_back(wl);
        mw.b.push_back(bl);
    }
    ops::BandPlan plan(dims, dim, &sw, &mw);
    auto xin = randn((size_t)rows * ftot, 1.0f, 77);
    Tensor feats = plan.band_split(dev(xin, {B, T, ftot}, DType::Float32));
    expect(feats.shape() == std::vector<int64_t>({B, T, nb, dim}), "band_split -> [B, T, nb, dim]");
    std::vector<float> rf((size_t)rows * nb * dim), rm((size_t)rows * ftot);
    orc_band_split(xin.data(), rows, dims.data(), nb, gcat.data(), wcat.data(), bcat.data(),
                   rf.data(), dim);
    check_close("band_split", feats, rf, 2e-2);
    Tensor m = plan.mask_estimator(feats);
    expect(m.shape() == std::vector<int64_t>({B, T, ftot}), "mask_estimator -> [B, T, sum dims]");
    const std::vector<float> fh = feats.to_cpu_f32();
    orc_mask_estimator(fh.data(), rows, dims.data(), nb, dim, hid, L, mwcat.data(), mbcat.data(),
                       rm.data());
    check_close("mask_estimator", m, rm, 2e-2);
    expect_throw("BandPlan with an fp32 matrix", [&] {
        ops::BandSplitWeights bad = sw;
        bad.w[0] = bad.w[0].to_f32();
        ops::BandPlan p(dims, dim, &bad, nullptr);
    });
    expect_throw("mask_estimator on the wrong band count",
                 [&] { plan.mask_estimator(Tensor::zeros({rows, nb + 1, dim})); });

    // STFT side: overlapping bands over 9 stereo bins, gather then merge.
    {
        const int F = 9, ch = 2, Tn = 5, Bb = 2, stems = 2;
        ops::StftBands sb;
        sb.channels = ch;
        sb.stft_bins = F;
        std::vector<int> bd;
        for (int lo : {0, 3, 5}) {  // bands over bins [0,4), [3,6), [5,9)
            const int hi = lo == 0 ? 4 : lo == 3 ? 6 : 9;
            for (int f = lo; f < hi; ++f)
                for (int s2 = 0; s2 < ch; ++s2) sb.freq_indices.push_back(f * ch + s2);
            bd.push_back(2 * (hi - lo) * ch);
        }
        ops::BandPlan sp(bd, 64, nullptr, nullptr, &sb);
        const int n = (int)sb.freq_indices.size();
        auto st = randn((size_t)Bb * ch * F * Tn * 2, 1.0f, 91);
        Tensor std_ = dev(st, {Bb * ch, F, Tn, 2}, DType::Float32);
        std::vector<float> rg((size_t)Bb * Tn * 2 * n);
        orc_band_gather(st.data(), Bb, ch, F, Tn, sb.freq_indices.data(), n, rg.data());
        check_close("band_gather", sp.band_gather(std_, Bb), rg, 0.0);
        auto mk = randn((size_t)stems * Bb * Tn * 2 * n, 1.0f, 92);
        std::vector<float> rm((size_t)Bb * stems * ch * F * Tn * 2);
        orc_mask_merge(mk.data(), stems, st.data(), Bb, ch, F, Tn, sb.freq_indices.data(), n, 1,
                       rm.data());
        check_close("mask_merge", sp.mask_merge(dev(mk, {stems, Bb, Tn, 2 * n}, DType::Float32),
                                               std_, Bb, true),
                    rm, 1e-6);
    }
}

static void test_stft() {
    // ops::stft / istft / hann_window (ops.h:87-96) against the oracle.
    const int n_fft = 256, hop = 64;
    const int64_t B = 2, L = 3000;
    Tensor w = ops::hann_window(n_fft);
    std::vector<float> wr(n_fft);
    orc_hann_window(wr.data(), n_fft);
    check_close("hann_window", w, wr, 1e-6);
    auto x = randn((size_t)(B * L), 1.0f, 61);
    Tensor s = ops::stft(dev(x, {B, L}, DType::Float32), n_fft, hop, n_fft, w);
    const int64_t T = (L + n_fft - n_fft) / hop + 1, F = n_fft / 2 + 1;
    expect(s.shape() == std::vector<int64_t>({B, F, T, 2}), "stft -> [B, F, T, 2]");
    std::vector<float> rs((size_t)(B * F * T * 2));
    orc_stft(x.data(), B, L, n_fft, hop, wr.data(), 1, 0, rs.data());
    check_close("stft", s, rs, 1e-5);
    Tensor y = ops::istft(s, n_fft, hop, n_fft, w, L);
    expect(y.shape() == std::vector<int64_t>({B, L}), "istft -> [B, length]");
    std::vector<float> ry((size_t)(B * L));
    const std::vector<float> sh = s.to_cpu_f32();
    orc_istft(sh.data(), B, T, n_fft, hop, wr.data(), L, 1, 0, ry.data());
    check_close("istft", y, ry, 1e-5);
    Tensor s1 = ops::stft(dev(x, {L}, DType::Float32), n_fft, hop, n_fft, w);  // 1-D signal
    expect(s1.shape() == std::vector<int64_t>({1, F, T, 2}), "stft of [L] -> [1, F, T, 2]");
    expect_throw("stft with win_length != n_fft",
                 [&] { ops::stft(dev(x, {B, L}, DType::Float32), n_fft, hop, 200, w); });
}

int main() {
    try {
        test_tensor();
        test_linear();
        test_rms_norm();
        test_rope_attention();
        test_stack();
        test_bands();
        test_stft();
        cudasep::CudaContext::instance().sync();
    } catch (const std::exception& ex) {
        std::printf("FAIL: uncaught exception: %s\n", ex.what());
        return 2;
    }
    std::printf("%s: %d checks, %d failed\n", g_fail ? "FAILED" : "OK", g_checks, g_fail);
    return g_fail ? 1 : 0;
}
