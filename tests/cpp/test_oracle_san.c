/*
 * test_oracle_san.c — every function of the CPU oracle (oracle/msst_oracle.h)
 * run at small, ragged sizes, for the host AddressSanitizer /
 * UndefinedBehaviorSanitizer build (`make sanitize`, CPU only).  Each call
 * is also checked against a closed form, so the run is a test, not only a
 * memory check:
 *   linear with identity W and bias; sigmoid(0) = 1/2; RMSNorm of a constant
 *   row; RoPE table at position 0 and the rotation there (identity);
 *   attention with Q = 0 (mean of V); split / gate-merge round trip; GLU
 *   with a zero gate half; band split of one band against norm + linear;
 *   STFT -> iSTFT round trip; Hann window symmetry; mel filterbank rows
 *   non-negative; transformer, stack, mask estimator, gather and merge
 *   finite (their values are pinned by the Python oracle tests).
 * Exit status 0 on success; the sanitizers abort on the first finding.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "msst_oracle.h"

static int failures = 0;

static void check(int ok, const char* what) {
    if (!ok) {
        fprintf(stderr, "FAIL %s\n", what);
        ++failures;
    }
}

static float* rnd(int64_t n, unsigned* seed, float scale) {
    float* p = (float*)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
    for (int64_t i = 0; i < n; ++i) {
        *seed = *seed * 1664525u + 1013904223u;
        p[i] = scale * (((float)(*seed >> 8) / 16777216.0f) * 2.0f - 1.0f);
    }
    return p;
}

static int all_finite(const float* p, int64_t n) {
    for (int64_t i = 0; i < n; ++i)
        if (!isfinite(p[i])) return 0;
    return 1;
}

static float max_abs_diff(const float* a, const float* b, int64_t n) {
    float m = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        const float d = fabsf(a[i] - b[i]);
        if (d > m) m = d;
    }
    return m;
}

static void test_linear(unsigned* seed) {
    const int64_t M = 7, K = 13;
    float* x = rnd(M * K, seed, 1.0f);
    float* b = rnd(K, seed, 1.0f);
    float* w = (float*)calloc((size_t)(K * K), sizeof(float));
    for (int64_t i = 0; i < K; ++i) w[i * K + i] = 1.0f;
    float* out = (float*)malloc(sizeof(float) * (size_t)(M * K));
    float* ref = (float*)malloc(sizeof(float) * (size_t)(M * K));
    orc_linear(x, w, b, NULL, out, M, K, K, ORC_ACT_NONE);
    for (int64_t r = 0; r < M; ++r)
        for (int64_t c = 0; c < K; ++c) ref[r * K + c] = x[r * K + c] + b[c];
    check(max_abs_diff(out, ref, M * K) < 1e-6f, "linear identity + bias");
    /* residual in place: out = x + (x + b) */
    memcpy(out, x, sizeof(float) * (size_t)(M * K));
    orc_linear(x, w, b, out, out, M, K, K, ORC_ACT_NONE);
    for (int64_t i = 0; i < M * K; ++i) ref[i] += x[i];
    check(max_abs_diff(out, ref, M * K) < 1e-5f, "linear residual in place");
    free(x); free(b); free(w); free(out); free(ref);
}

static void test_activation(void) {
    float z[3] = {0.0f, 0.0f, 0.0f}, o[3];
    orc_activation(z, o, 3, ORC_ACT_SIGMOID);
    check(fabsf(o[0] - 0.5f) < 1e-7f && fabsf(o[2] - 0.5f) < 1e-7f, "sigmoid(0)");
    orc_activation(z, o, 3, ORC_ACT_GELU);
    check(o[1] == 0.0f, "gelu(0)");
    orc_activation(z, o, 3, ORC_ACT_TANH);
    check(o[0] == 0.0f, "tanh(0)");
}

static void test_rms_norm(void) {
    const int64_t rows = 3, D = 5;
    float x[15], g[5], out[15];
    for (int i = 0; i < 15; ++i) x[i] = 2.0f;
    for (int i = 0; i < 5; ++i) g[i] = 1.0f;
    orc_rms_norm(x, g, 3.0f, out, rows, D);
    const float want = 2.0f / sqrtf(4.0f * D + 1e-12f) * 3.0f;
    int ok = 1;
    for (int i = 0; i < 15; ++i) ok &= fabsf(out[i] - want) < 1e-6f;
    check(ok, "rms_norm constant row");
}

static void test_rope(unsigned* seed) {
    const int n = 9, dh = 64;
    float* c = (float*)malloc(sizeof(float) * n * dh / 2);
    float* s = (float*)malloc(sizeof(float) * n * dh / 2);
    orc_rope_table(n, dh, c, s);
    int ok = 1;
    for (int i = 0; i < dh / 2; ++i) ok &= c[i] == 1.0f && s[i] == 0.0f;
    check(ok, "rope table at position 0");
    const int64_t B = 2, H = 3, N = 1, D = 64;
    float* q = rnd(B * H * N * D, seed, 1.0f);
    float* k = rnd(B * H * N * D, seed, 1.0f);
    float* q0 = (float*)malloc(sizeof(float) * (size_t)(B * H * N * D));
    memcpy(q0, q, sizeof(float) * (size_t)(B * H * N * D));
    orc_rope_apply(q, k, c, s, B, H, N, D);
    check(max_abs_diff(q, q0, B * H * N * D) == 0.0f, "rope identity at position 0");
    free(c); free(s); free(q); free(k); free(q0);
}

static void test_attention_layout(unsigned* seed) {
    const int64_t B = 2, H = 3, N = 5, Nk = 7, D = 64;
    float* q = (float*)calloc((size_t)(B * H * N * D), sizeof(float));
    float* k = rnd(B * H * Nk * D, seed, 1.0f);
    float* v = rnd(B * H * Nk * D, seed, 1.0f);
    float* o = (float*)malloc(sizeof(float) * (size_t)(B * H * N * D));
    orc_attention(q, k, v, o, B, H, N, Nk, D, 0.125f);
    int ok = 1;
    for (int64_t bh = 0; bh < B * H; ++bh)
        for (int64_t d = 0; d < D; ++d) {
            float mean = 0.0f;
            for (int64_t j = 0; j < Nk; ++j) mean += v[(bh * Nk + j) * D + d];
            mean /= (float)Nk;
            for (int64_t i = 0; i < N; ++i) ok &= fabsf(o[(bh * N + i) * D + d] - mean) < 1e-5f;
        }
    check(ok, "attention with Q = 0 is the mean of V");
    /* split -> gate-merge with unit gates is the (q) column block of qkv */
    float* qkv = rnd(B * N * 3 * H * D, seed, 1.0f);
    float* qs = (float*)malloc(sizeof(float) * (size_t)(B * H * N * D));
    float* ks = (float*)malloc(sizeof(float) * (size_t)(B * H * N * D));
    float* vs = (float*)malloc(sizeof(float) * (size_t)(B * H * N * D));
    float* gates = (float*)malloc(sizeof(float) * (size_t)(B * N * H));
    float* merged = (float*)malloc(sizeof(float) * (size_t)(B * N * H * D));
    for (int64_t i = 0; i < B * N * H; ++i) gates[i] = 1.0f;
    orc_split_qkv(qkv, qs, ks, vs, B, N, H, D);
    orc_gate_merge(qs, gates, merged, B, H, N, D);
    ok = 1;
    for (int64_t t = 0; t < B * N; ++t)
        for (int64_t c = 0; c < H * D; ++c) ok &= merged[t * H * D + c] == qkv[t * 3 * H * D + c];
    check(ok, "split / merge round trip");
    free(q); free(k); free(v); free(o); free(qkv); free(qs); free(ks); free(vs); free(gates);
    free(merged);
}

static void make_layer(orc_layer_weights* w, float** keep, int64_t dim, int64_t H, int64_t Dh,
                       int64_t ff, int final_norm, unsigned* seed) {
    const int64_t HD = H * Dh;
    keep[0] = rnd(dim, seed, 0.02f);
    for (int64_t i = 0; i < dim; ++i) keep[0][i] += 1.0f;
    keep[1] = rnd(3 * HD * dim, seed, 0.05f);
    keep[2] = rnd(H * dim, seed, 0.05f);
    keep[3] = rnd(H, seed, 0.05f);
    keep[4] = rnd(dim * HD, seed, 0.05f);
    keep[5] = rnd(dim, seed, 0.02f);
    for (int64_t i = 0; i < dim; ++i) keep[5][i] += 1.0f;
    keep[6] = rnd(ff * dim, seed, 0.05f);
    keep[7] = rnd(ff, seed, 0.05f);
    keep[8] = rnd(dim * ff, seed, 0.05f);
    keep[9] = rnd(dim, seed, 0.05f);
    keep[10] = final_norm ? rnd(dim, seed, 0.02f) : NULL;
    w->attn_gamma = keep[0]; w->w_qkv = keep[1]; w->w_gate = keep[2]; w->b_gate = keep[3];
    w->w_out = keep[4]; w->ff_gamma = keep[5]; w->w_ff1 = keep[6]; w->b_ff1 = keep[7];
    w->w_ff2 = keep[8]; w->b_ff2 = keep[9]; w->final_gamma = keep[10];
}

static void test_transformer_stack(unsigned* seed) {
    const int64_t B = 1, T = 5, F = 3, dim = 32, H = 2, Dh = 64, ff = 48, depth = 2;
    orc_layer_weights layers[4];
    float* keep[4][11];
    for (int i = 0; i < 4; ++i) make_layer(&layers[i], keep[i], dim, H, Dh, ff, i % 2, seed);
    float* x = rnd(B * T * F * dim, seed, 1.0f);
    float* c = (float*)malloc(sizeof(float) * T * Dh / 2);
    float* s = (float*)malloc(sizeof(float) * T * Dh / 2);
    orc_rope_table((int)T, (int)Dh, c, s);
    orc_transformer(x, B * F, T, dim, H, Dh, ff, &layers[0], c, s);
    check(all_finite(x, B * T * F * dim), "transformer finite");
    float* g = rnd(dim, seed, 0.02f);
    orc_roformer_stack(x, B, T, F, dim, H, Dh, ff, depth, layers, g);
    check(all_finite(x, B * T * F * dim), "stack finite");
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 11; ++j) free(keep[i][j]);
    free(x); free(c); free(s); free(g);
}

static void test_bands(unsigned* seed) {
    const int dims[3] = {4, 6, 2};
    const int nb = 3;
    const int64_t rows = 5, dim = 8, hid = 12, sumd = 12;
    float* x = rnd(rows * sumd, seed, 1.0f);
    float* gamma = rnd(sumd, seed, 0.1f);
    for (int i = 0; i < sumd; ++i) gamma[i] += 1.0f;
    float* w = rnd(dim * sumd, seed, 0.2f);
    float* bias = rnd(nb * dim, seed, 0.1f);
    float* out = (float*)malloc(sizeof(float) * (size_t)(rows * nb * dim));
    orc_band_split(x, rows, dims, nb, gamma, w, bias, out, dim);
    /* band 1 alone (columns 4..9) against rms_norm + linear */
    float xb[30], yb[30], ob[40];
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < 6; ++j) xb[r * 6 + j] = x[r * sumd + 4 + j];
    orc_rms_norm(xb, gamma + 4, sqrtf(6.0f), yb, rows, 6);
    orc_linear(yb, w + dim * 4, bias + dim, NULL, ob, rows, 6, dim, ORC_ACT_NONE);
    int ok = 1;
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < dim; ++j) ok &= fabsf(out[(r * nb + 1) * dim + j] - ob[r * dim + j]) < 1e-5f;
    check(ok, "band split band 1 = norm + linear");
    /* mask estimator, 2 layers: widths dim -> hid -> 2 d_b per band */
    int64_t wn = 0, bn = 0;
    for (int b = 0; b < nb; ++b) {
        wn += hid * dim + 2 * dims[b] * hid;
        bn += hid + 2 * dims[b];
    }
    float* mw = rnd(wn, seed, 0.2f);
    float* mb = rnd(bn, seed, 0.1f);
    float* est = (float*)malloc(sizeof(float) * (size_t)(rows * sumd));
    orc_mask_estimator(out, rows, dims, nb, dim, hid, 2, mw, mb, est);
    check(all_finite(est, rows * sumd), "mask estimator finite");
    /* GLU with a zero gate half: out = x / 2 */
    float gx[8] = {1, -2, 3, -4, 0, 0, 0, 0}, go[4];
    orc_glu(gx, go, 1, 4);
    check(go[0] == 0.5f && go[1] == -1.0f && go[3] == -2.0f, "glu with zero gates");
    free(x); free(gamma); free(w); free(bias); free(out); free(mw); free(mb); free(est);
}

static void test_gather_merge(unsigned* seed) {
    const int64_t B = 1, ch = 2, F = 5, T = 3, stems = 2;
    const int fidx[6] = {0, 3, 4, 9, 1, 3};
    const int64_t n = 6;
    float* stft = rnd(B * ch * F * T * 2, seed, 1.0f);
    float* feat = (float*)malloc(sizeof(float) * (size_t)(B * T * 2 * n));
    orc_band_gather(stft, B, ch, F, T, fidx, n, feat);
    check(all_finite(feat, B * T * 2 * n), "band gather finite");
    float* masks = rnd(stems * B * T * 2 * n, seed, 1.0f);
    float* out = (float*)malloc(sizeof(float) * (size_t)(B * stems * ch * F * T * 2));
    orc_mask_merge(masks, stems, stft, B, ch, F, T, fidx, n, 1, out);
    check(all_finite(out, B * stems * ch * F * T * 2), "mask merge finite");
    free(stft); free(feat); free(masks); free(out);
}

static void test_stft(unsigned* seed) {
    const int n_fft = 16, hop = 4;
    const int64_t B = 2, L = 61;
    float win[16];
    orc_hann_window(win, n_fft);
    int ok = win[0] == 0.0f;
    for (int i = 1; i < n_fft; ++i) ok &= fabsf(win[i] - win[n_fft - i]) < 1e-6f;
    check(ok, "hann window periodic symmetry");
    const int64_t T = (L + n_fft - n_fft) / hop + 1;
    float* sig = rnd(B * L, seed, 1.0f);
    float* spec = (float*)malloc(sizeof(float) * (size_t)(B * (n_fft / 2 + 1) * T * 2));
    float* back = (float*)malloc(sizeof(float) * (size_t)(B * L));
    orc_stft(sig, B, L, n_fft, hop, win, 1, 0, spec);
    orc_istft(spec, B, T, n_fft, hop, win, L, 1, 0, back);
    /* frames cover [0, (T - 1) hop) of the centred signal; the rest of
     * `length` is zero-padded, as torch.istft does */
    const int64_t hi = (T - 1) * hop < L ? (T - 1) * hop : L;
    float err = 0.0f;
    for (int64_t b = 0; b < B; ++b) {
        const float e = max_abs_diff(sig + b * L, back + b * L, hi);
        if (e > err) err = e;
        for (int64_t i = hi; i < L; ++i) err = fmaxf(err, fabsf(back[b * L + i]));
    }
    check(err < 1e-4f, "stft -> istft round trip");
    float* mel = (float*)malloc(sizeof(float) * 7 * (n_fft / 2 + 1));
    orc_mel_filterbank(mel, 8000, n_fft, 7, 0.0f, 0.0f);
    ok = 1;
    for (int i = 0; i < 7 * (n_fft / 2 + 1); ++i) ok &= mel[i] >= 0.0f && isfinite(mel[i]);
    check(ok, "mel filterbank non-negative");
    free(sig); free(spec); free(back); free(mel);
}

int main(void) {
    unsigned seed = 12345u;
    orc_set_num_threads(2);
    test_linear(&seed);
    test_activation();
    test_rms_norm();
    test_rope(&seed);
    test_attention_layout(&seed);
    test_transformer_stack(&seed);
    test_bands(&seed);
    test_gather_merge(&seed);
    test_stft(&seed);
    if (failures) {
        fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    printf("oracle sanitizer run: all checks passed\n");
    return 0;
}
