// test_tensor_views.cpp — the reference Tensor view surface on the GPU and
// the reference's own per-op Roformer call sequence written against it.
//
// Part 1: permute / transpose / slice / split / unbind / expand / cat /
// stack / broadcast operators / in-place forms / squeeze / reshape of views
// against the same index arithmetic on the host (exact: these are copies and
// single fp32 operations).
// Part 2: apply_attention / apply_feedforward / apply_transformer /
// compute_rotary_cos_sin of model_bs_roformer.cu:205-331 and the depth
// loop's axis permutes (:482-534), each step the reference's ops / Tensor
// call, on [62 bands, 801 frames, 512] against the CPU oracle's transformer
// (orc_transformer / orc_roformer_stack) on the same seeded weights:
// normwise max|y - r| / max|r| <= 1e-4 with fp32 weights, <= 2e-2 with fp16
// weights (activations rounded to fp16 at every GEMM).
// Exit status 0 and a last line "OK: ..." when every check passes.
#include <hip/hip_fp16.h>

#include <cmath>
#include <cstdio>
#include <functional>
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

static Tensor dev(const std::vector<float>& v, std::vector<int64_t> shape,
                  DType dt = DType::Float32) {
    return Tensor::from_cpu_f32(v.data(), shape).to_dtype(dt);
}

static int64_t numel(const std::vector<int64_t>& s) {
    int64_t n = 1;
    for (int64_t x : s) n *= x;
    return n;
}

// Host gather: out[i] = src[offset(i)] over `shape` in row-major order, the
// offset from element strides.
static std::vector<float> gather(const std::vector<float>& src, const std::vector<int64_t>& shape,
                                 const std::vector<int64_t>& strides, int64_t base = 0) {
    const int n = (int)shape.size();
    std::vector<float> out;
    std::vector<int64_t> c(n, 0);
    for (int64_t i = 0; i < numel(shape); ++i) {
        int64_t o = base;
        for (int d = 0; d < n; ++d) o += c[d] * strides[d];
        out.push_back(src[o]);
        for (int d = n - 1; d >= 0; --d) {
            if (++c[d] < shape[d]) break;
            c[d] = 0;
        }
    }
    return out;
}

static std::vector<int64_t> rowmajor(const std::vector<int64_t>& s) {
    std::vector<int64_t> st(s.size());
    int64_t a = 1;
    for (int d = (int)s.size() - 1; d >= 0; --d) {
        st[d] = a;
        a *= s[d];
    }
    return st;
}

static void expect_equal(const std::string& name, const Tensor& t, const std::vector<float>& r,
                         const std::vector<int64_t>& shape) {
    const std::vector<float> h = t.to_cpu_f32();
    bool ok = t.shape() == shape && h == r;
    expect(ok, name + " (shape " + t.shape_str() + ")");
}

static double rel_err(const std::vector<float>& y, const std::vector<float>& r) {
    double num = 0, den = 0;
    for (size_t i = 0; i < r.size(); ++i) {
        num = std::fmax(num, std::fabs((double)y[i] - r[i]));
        den = std::fmax(den, std::fabs((double)r[i]));
    }
    if (!std::isfinite(num) || y.size() != r.size()) return INFINITY;
    return den > 0 ? num / den : num;
}

static void check_close(const std::string& name, const Tensor& y, const std::vector<float>& r,
                        double tol) {
    const double e = rel_err(y.to_cpu_f32(), r);
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s: rel err %.3e (tol %.1e)", name.c_str(), e, tol);
    std::printf("%s\n", buf);
    expect(e <= tol, buf);
}

// ---------------------------------------------------------------------------
// Part 1: views
// ---------------------------------------------------------------------------
static void test_views(DType dt) {
    const std::string tag = dt == DType::Float16 ? " f16" : " f32";
    const std::vector<int64_t> s = {2, 3, 4, 5};
    // Values exact in fp16 (small integers / 8).
    std::vector<float> v(numel(s));
    for (size_t i = 0; i < v.size(); ++i) v[i] = (float)((int)(i * 7 % 61) - 30) / 8.0f;
    Tensor x = dev(v, s, dt);
    const std::vector<int64_t> rs = rowmajor(s);
    expect(x.is_contiguous(), "fresh tensor is contiguous" + tag);

    // permute (view) then contiguous (one strided copy)
    Tensor p = x.permute({2, 0, 3, 1});
    expect(!p.is_contiguous() && p.data_ptr() == x.data_ptr(), "permute is a view" + tag);
    const std::vector<int64_t> ps = {4, 2, 5, 3}, pst = {rs[2], rs[0], rs[3], rs[1]};
    expect_equal("permute.contiguous" + tag, p.contiguous(), gather(v, ps, pst), ps);
    expect_equal("permute.reshape copies" + tag, p.reshape({8, 15}), gather(v, ps, pst), {8, 15});
    expect_equal("transpose(-1, 1)" + tag, x.transpose(-1, 1).contiguous(),
                 gather(v, {2, 5, 4, 3}, {rs[0], rs[3], rs[2], rs[1]}), {2, 5, 4, 3});

    // slice / split / unbind
    Tensor sl = x.slice(2, 1, -1);  // [2, 3, 2, 5]
    expect(sl.data_ptr() != x.data_ptr() && !sl.is_contiguous(), "slice is an offset view" + tag);
    expect_equal("slice(2, 1, -1)" + tag, sl.contiguous(), gather(v, {2, 3, 2, 5}, rs, rs[2]),
                 {2, 3, 2, 5});
    expect(x.slice(1, 2, 2).is_empty(), "empty slice" + tag);
    expect(x.slice(3, -2, 100).size(3) == 2, "slice clamps the end" + tag);
    std::vector<Tensor> parts = x.split(3, {1, 3, 1});
    expect(parts.size() == 3 && parts[1].size(3) == 3, "split sizes" + tag);
    expect_equal("split[1]" + tag, parts[1].contiguous(), gather(v, {2, 3, 4, 3}, rs, 1),
                 {2, 3, 4, 3});
    expect_throw("split with a bad total" + tag, [&] { x.split(3, {2, 2}); });
    std::vector<Tensor> ub = x.unbind(1);
    expect(ub.size() == 3, "unbind count" + tag);
    expect_equal("unbind[2]" + tag, ub[2], gather(v, {2, 4, 5}, {rs[0], rs[2], rs[3]}, 2 * rs[1]),
                 {2, 4, 5});

    // squeeze / unsqueeze
    expect_throw("squeeze of a non-1 axis" + tag, [&] { x.squeeze(1); });
    Tensor q = x.slice(0, 1, 2).squeeze(0);
    expect_equal("slice.squeeze" + tag, q, gather(v, {3, 4, 5}, {rs[1], rs[2], rs[3]}, rs[0]),
                 {3, 4, 5});
    expect(x.unsqueeze(-1).shape() == std::vector<int64_t>({2, 3, 4, 5, 1}), "unsqueeze(-1)" + tag);

    // expand (stride 0) and its contiguous copy
    Tensor row = dev(std::vector<float>{1, 2, 3, 4, 5}, {5}, dt);
    Tensor ex = row.expand({3, 5});
    expect(ex.strides()[0] == 0, "expand gives stride 0" + tag);
    expect_equal("expand.contiguous" + tag, ex.contiguous(),
                 {1, 2, 3, 4, 5, 1, 2, 3, 4, 5, 1, 2, 3, 4, 5}, {3, 5});
    expect_throw("expand of a non-1 axis" + tag, [&] { x.expand({2, 3, 4, 6}); });

    // cat / stack (views as inputs)
    Tensor c = Tensor::cat({parts[2], parts[0], parts[1]}, -1);
    std::vector<float> cr;
    for (int64_t r = 0; r < 24; ++r) {
        cr.push_back(v[r * 5 + 4]);
        cr.push_back(v[r * 5 + 0]);
        for (int j = 1; j < 4; ++j) cr.push_back(v[r * 5 + j]);
    }
    expect_equal("cat of split views" + tag, c, cr, s);
    Tensor st = Tensor::stack({ub[0], ub[1], ub[2]}, 0);  // [3, 2, 4, 5]
    expect_equal("stack(unbind(1), 0)" + tag, st, gather(v, {3, 2, 4, 5}, {rs[1], rs[0], rs[2], rs[3]}),
                 {3, 2, 4, 5});
    Tensor st2 = Tensor::stack({x, x}, 2);  // [2, 3, 2, 4, 5]
    std::vector<float> s2r;
    for (int64_t a = 0; a < 6; ++a)
        for (int k = 0; k < 2; ++k)
            for (int64_t e = 0; e < 20; ++e) s2r.push_back(v[a * 20 + e]);
    expect_equal("stack at an inner axis" + tag, st2, s2r, {2, 3, 2, 4, 5});
    expect_throw("cat with a shape mismatch" + tag, [&] { Tensor::cat({x, parts[0]}, 0); });

    // broadcast operators on views
    const std::vector<int64_t> gs = {2, 4, 3};  // [B, N, H] gates
    std::vector<float> gv(numel(gs));
    for (size_t i = 0; i < gv.size(); ++i) gv[i] = (float)((int)(i % 5) - 2) / 4.0f;
    Tensor gates = dev(gv, gs, dt).permute({0, 2, 1}).unsqueeze(-1);  // [B, H, N, 1]
    Tensor att = x.permute({0, 1, 2, 3});                              // [2, 3, 4, 5]
    std::vector<float> mr(v.size());
    for (int64_t b = 0; b < 2; ++b)
        for (int64_t h = 0; h < 3; ++h)
            for (int64_t n = 0; n < 4; ++n)
                for (int64_t d = 0; d < 5; ++d) {
                    const int64_t i = ((b * 3 + h) * 4 + n) * 5 + d;
                    mr[i] = v[i] * gv[(b * 4 + n) * 3 + h];
                }
    expect_equal("out * gates broadcast" + tag, att * gates, mr, s);
    std::vector<float> ar(v.size()), dr(v.size()), sr2(v.size());
    for (size_t i = 0; i < v.size(); ++i) {
        ar[i] = v[i] + v[i % 5];
        sr2[i] = v[i] - v[i % 5];
        dr[i] = v[i] / 2.0f;
    }
    Tensor lastrow = x.slice(0, 0, 1).slice(1, 0, 1).slice(2, 0, 1);  // [1,1,1,5] view
    expect_equal("x + broadcast row" + tag, x + lastrow, ar, s);
    expect_equal("x - broadcast row" + tag, x - lastrow, sr2, s);
    expect_equal("x / full(2)" + tag, x / Tensor::full({1}, 2.0f, dt), dr, s);
    Tensor y = x.clone();
    y.add_(lastrow);
    expect_equal("add_ broadcast" + tag, y, ar, s);
    Tensor pv = x.clone().permute({1, 0, 2, 3});  // in place on a view
    pv.add_(Tensor::ones({5}, dt));
    std::vector<float> p1;
    for (float e : gather(v, {3, 2, 4, 5}, {rs[1], rs[0], rs[2], rs[3]})) p1.push_back(e + 1.0f);
    expect_equal("add_ on a permuted view" + tag, pv, p1, {3, 2, 4, 5});
    Tensor z = x.clone();
    z.mul_(Tensor::full({4, 1}, 0.5f, dt));
    std::vector<float> hr;
    for (float e : v) hr.push_back(e * 0.5f);
    expect_equal("mul_ broadcast [4,1]" + tag, z, hr, s);
    expect_throw("add_ that would grow the tensor" + tag,
                 [&] { Tensor t = parts[0].contiguous(); t.add_(x); });
    expect_throw("dtype mismatch" + tag, [&] {
        (void)(x * dev(v, s, dt == DType::Float16 ? DType::Float32 : DType::Float16));
    });

    // complex_mul / index_fill (the forward's mask side, model_bs_roformer.cu:569, :589)
    {
        Tensor a = x.reshape({60, 2}), b = x.permute({3, 2, 1, 0}).contiguous().reshape({60, 2});
        const std::vector<float> ah = a.to_cpu_f32(), bh = b.to_cpu_f32();
        std::vector<float> cr(120);
        for (int i = 0; i < 60; ++i) {
            cr[2 * i] = ah[2 * i] * bh[2 * i] - ah[2 * i + 1] * bh[2 * i + 1];
            cr[2 * i + 1] = ah[2 * i] * bh[2 * i + 1] + ah[2 * i + 1] * bh[2 * i];
        }
        if (dt == DType::Float16)
            for (auto& e : cr) e = __half2float(__float2half(e));
        Tensor cm = ops::complex_mul(a, b);
        expect(cm.dtype() == dt, "complex_mul keeps a's dtype" + tag);
        expect_equal("complex_mul" + tag, cm, cr, {60, 2});
        std::vector<float> fr = v;
        for (int64_t i = 0; i < (int64_t)v.size(); ++i)
            if ((i / rs[1]) % 3 == 1) fr[i] = -2.5f;
        expect_equal("index_fill(dim 1, 1, -2.5)" + tag, ops::index_fill(x, 1, 1, -2.5f), fr, s);
        expect_equal("index_fill leaves x" + tag, x, v, s);
        expect_throw("index_fill out of range" + tag, [&] { ops::index_fill(x, 1, 3, 0.0f); });
    }

    // ops accept views: rms_norm of a split view (the band split pattern)
    Tensor gamma = dev(std::vector<float>(3, 1.0f), {3});
    check_close("rms_norm of a split view" + tag, ops::rms_norm(parts[1], gamma, std::sqrt(3.0f)),
                ops::rms_norm(parts[1].contiguous(), gamma, std::sqrt(3.0f)).to_cpu_f32(), 0.0);
}

// ---------------------------------------------------------------------------
// Part 2: the reference's per-op Roformer sequence on this surface.
// ---------------------------------------------------------------------------
struct Layer {
    std::vector<float> attn_gamma, w_qkv, w_gate, b_gate, w_out, ff_gamma, w_ff1, b_ff1, w_ff2,
        b_ff2;
};
struct DevLayer {
    Tensor attn_gamma, w_qkv, w_gate, b_gate, w_out, ff_gamma, w_ff1, b_ff1, w_ff2, b_ff2;
};

static Layer make_layer(int64_t dim, int64_t H, int64_t Dh, int64_t ff, uint64_t seed, bool f16) {
    const int64_t hd = H * Dh;
    auto w = [&](size_t n, uint64_t k) {
        auto r = randn(n, 0.02f, seed * 100 + k);
        return f16 ? round16(r) : r;
    };
    Layer L;
    L.attn_gamma = randn(dim, 0.02f, seed * 100 + 1, 1.0f);
    L.w_qkv = w(3 * hd * dim, 2);
    L.w_gate = w(H * dim, 3);
    L.b_gate = randn(H, 0.02f, seed * 100 + 4);
    L.w_out = w(dim * hd, 5);
    L.ff_gamma = randn(dim, 0.02f, seed * 100 + 6, 1.0f);
    L.w_ff1 = w(ff * dim, 7);
    L.b_ff1 = randn(ff, 0.02f, seed * 100 + 8);
    L.w_ff2 = w(dim * ff, 9);
    L.b_ff2 = randn(dim, 0.02f, seed * 100 + 10);
    return L;
}

static DevLayer upload(const Layer& L, int64_t dim, int64_t H, int64_t Dh, int64_t ff, DType wdt) {
    const int64_t hd = H * Dh;
    DevLayer d;
    d.attn_gamma = dev(L.attn_gamma, {dim});
    d.w_qkv = dev(L.w_qkv, {3 * hd, dim}, wdt);
    d.w_gate = dev(L.w_gate, {H, dim}, wdt);
    d.b_gate = dev(L.b_gate, {H});
    d.w_out = dev(L.w_out, {dim, hd}, wdt);
    d.ff_gamma = dev(L.ff_gamma, {dim});
    d.w_ff1 = dev(L.w_ff1, {ff, dim}, wdt);
    d.b_ff1 = dev(L.b_ff1, {ff});
    d.w_ff2 = dev(L.w_ff2, {dim, ff}, wdt);
    d.b_ff2 = dev(L.b_ff2, {dim});
    return d;
}

static orc_layer_weights orc_view(const Layer& L) {
    orc_layer_weights w{};
    w.attn_gamma = L.attn_gamma.data();
    w.w_qkv = L.w_qkv.data();
    w.w_gate = L.w_gate.data();
    w.b_gate = L.b_gate.data();
    w.w_out = L.w_out.data();
    w.ff_gamma = L.ff_gamma.data();
    w.w_ff1 = L.w_ff1.data();
    w.b_ff1 = L.b_ff1.data();
    w.w_ff2 = L.w_ff2.data();
    w.b_ff2 = L.b_ff2.data();
    w.final_gamma = nullptr;
    return w;
}

// model_bs_roformer.cu:205-230: host fp32 table, stacked [2, N, Dh/2]; the
// depth loop takes rows 0 and 1 (:496-503).
static void rotary_cos_sin(int seq_len, int dim, Tensor& cos_t, Tensor& sin_t) {
    const int half = dim / 2;
    std::vector<float> c((size_t)seq_len * half), s((size_t)seq_len * half);
    for (int n = 0; n < seq_len; ++n)
        for (int i = 0; i < half; ++i) {
            const float freq = 1.0f / std::pow(10000.0f, (float)(2 * i) / (float)dim);
            const float angle = (float)n * freq;
            c[(size_t)n * half + i] = std::cos(angle);
            s[(size_t)n * half + i] = std::sin(angle);
        }
    Tensor rot = Tensor::stack({Tensor::from_cpu_f32(c.data(), {seq_len, half}),
                                Tensor::from_cpu_f32(s.data(), {seq_len, half})},
                               0);
    cos_t = rot.slice(0, 0, 1).squeeze(0).contiguous();
    sin_t = rot.slice(0, 1, 2).squeeze(0).contiguous();
}

// model_bs_roformer.cu:236-284
static Tensor apply_attention(const Tensor& x, const DevLayer& w, int64_t H, int64_t Dh,
                              const Tensor& cos_f, const Tensor& sin_f) {
    const int64_t dim = x.size(-1);
    Tensor normed = ops::rms_norm(x, w.attn_gamma, std::sqrt((float)dim));
    Tensor qkv = ops::linear_no_bias(normed, w.w_qkv);
    const int64_t B = qkv.size(0), N = qkv.size(1);
    Tensor qkv_r = qkv.reshape({B, N, 3, H, Dh}).permute({2, 0, 3, 1, 4});
    Tensor q = qkv_r.slice(0, 0, 1).squeeze(0).contiguous();
    Tensor k = qkv_r.slice(0, 1, 2).squeeze(0).contiguous();
    Tensor v = qkv_r.slice(0, 2, 3).squeeze(0).contiguous();
    ops::apply_rotary_emb(q, k, cos_f, sin_f);
    Tensor out = ops::scaled_dot_product_attention(q, k, v, 1.0f / std::sqrt((float)Dh));
    Tensor gates = ops::linear_sigmoid(normed, w.w_gate, w.b_gate);
    gates = gates.permute({0, 2, 1}).unsqueeze(-1);
    out = out * gates;
    out = out.permute({0, 2, 1, 3}).contiguous();
    out = out.reshape({B, N, H * Dh});
    return ops::linear_no_bias(out, w.w_out);
}

// model_bs_roformer.cu:290-304
static Tensor apply_feedforward(const Tensor& x, const DevLayer& w) {
    Tensor h = ops::rms_norm(x, w.ff_gamma, std::sqrt((float)x.size(-1)));
    h = ops::linear_gelu(h, w.w_ff1, w.b_ff1);
    return ops::linear(h, w.w_ff2, w.b_ff2);
}

// model_bs_roformer.cu:310-331 (depth 1)
static Tensor apply_transformer(const Tensor& x, const DevLayer& w, int64_t H, int64_t Dh,
                                const Tensor& cos_f, const Tensor& sin_f) {
    Tensor out = x;
    out = out + apply_attention(out, w, H, Dh, cos_f, sin_f);
    out = out + apply_feedforward(out, w);
    return out;
}

static void test_reference_sequence(DType wdt) {
    const bool f16 = wdt == DType::Float16;
    const std::string tag = f16 ? " (fp16 W)" : " (fp32 W)";
    const double tol = f16 ? 2e-2 : 1e-4;
    const int64_t F = 62, T = 801, dim = 512, H = 8, Dh = 64, ff = 2048;
    const Layer lt = make_layer(dim, H, Dh, ff, 11, f16), lf = make_layer(dim, H, Dh, ff, 12, f16);
    const DevLayer dt_ = upload(lt, dim, H, Dh, ff, wdt), df = upload(lf, dim, H, Dh, ff, wdt);
    Tensor tcos, tsin, fcos, fsin;
    rotary_cos_sin((int)T, (int)Dh, tcos, tsin);
    rotary_cos_sin((int)F, (int)Dh, fcos, fsin);
    std::vector<float> tc(T * Dh / 2), ts(T * Dh / 2);
    orc_rope_table((int)T, (int)Dh, tc.data(), ts.data());
    expect(tcos.to_cpu_f32() == tc && tsin.to_cpu_f32() == ts,
           "stacked rotary table rows equal the oracle table" + tag);

    // One time transformer on [62 bands, 801 frames, 512] (the time layer's
    // [B*F, T, dim] after the depth loop's permute).
    const std::vector<float> x0 = randn((size_t)F * T * dim, 1.0f, 5);
    std::vector<float> ref = x0;
    const orc_layer_weights ot = orc_view(lt), of = orc_view(lf);
    orc_transformer(ref.data(), F, T, dim, H, Dh, ff, &ot, tc.data(), ts.data());
    Tensor x = dev(x0, {F, T, dim});
    check_close("reference per-op time transformer [62, 801, 512]" + tag,
                apply_transformer(x, dt_, H, Dh, tcos, tsin), ref, tol);

    // One depth of the reference's loop (:482-534) on x [1, T, F, dim]: the
    // permutes to and from [B*F, T, dim], the frequency layer on [B*T, F, dim].
    std::vector<float> sref = x0;  // read as [1, T, F, dim]
    const orc_layer_weights pair[2] = {ot, of};
    orc_roformer_stack(sref.data(), 1, T, F, dim, H, Dh, ff, 1, pair, nullptr);
    Tensor xs = dev(x0, {1, T, F, dim});
    xs = xs.permute({0, 2, 1, 3}).contiguous().reshape({F, T, dim});
    xs = apply_transformer(xs, dt_, H, Dh, tcos, tsin);
    xs = xs.reshape({1, F, T, dim}).permute({0, 2, 1, 3}).contiguous().reshape({T, F, dim});
    xs = apply_transformer(xs, df, H, Dh, fcos, fsin);
    check_close("reference per-op depth loop (time + frequency) [1, 801, 62, 512]" + tag,
                xs.reshape({1, T, F, dim}), sref, tol);
}

int main() {
    try {
        test_views(DType::Float32);
        test_views(DType::Float16);
        test_reference_sequence(DType::Float32);
        test_reference_sequence(DType::Float16);
    } catch (const std::exception& ex) {
        std::printf("FAIL: exception %s\n", ex.what());
        return 1;
    }
    if (g_fail) {
        std::printf("FAILED: %d of %d checks\n", g_fail, g_checks);
        return 1;
    }
    std::printf("OK: %d checks\n", g_checks);
    return 0;
}
