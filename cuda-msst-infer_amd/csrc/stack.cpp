// stack.cpp — the axial Roformer transformer stack driven natively through
// the C ABI (one stream, caller workspace, no allocation, no host sync).
//
// Reference: the depth loop of model_bs_roformer.cu:482-539 and
// model_mel_band_roformer.cu:843-906, each transformer being
// apply_attention + apply_feedforward (model_bs_roformer.cu:236-331,
// model_mel_band_roformer.cu:519-651).
//
// MI355X layout decision: the reference transposes the fp32 activation
// [B,T,F,dim] <-> [B,F,T,dim] twice per depth (permute().contiguous()).
// Every op of a transformer except attention is token-wise, so this driver
// keeps x in place in the caller's order [B,T,F,dim] for all 2*depth
// transformers and lets the attention kernel address either axis's
// sequences with token strides (msst_seq_layout):
//   time layer : sequence (b,f), position t -> token (b*T + t)*F + f
//   freq layer : sequence (b,t), position f -> token (b*T + t)*F + f
// (no transposes at all; an earlier version transposed once to [B,F,T,dim]
// on entry and once back on exit, 2 x 31 us per BSRoformer chunk).
// msst_roformer_transformer, the single-transformer entry, takes the
// time-major order [B,F,T,dim].
// Per transformer (fp16 weights):
//   rms_norm_gate   x(f32) -> xn(f16), gates(f32)   [HBM]
//   linear + RoPE   xn -> qkv(f16), q/k rotated      [MFMA]
//   attention       qkv -> merged(f16) (gate)        [MFMA]
//   linear + res    merged -> x += .                 [MFMA]
//   rms_norm        x -> xn(f16)                     [HBM]
//   linear + GELU   xn -> hidden(f16)                [MFMA]
//   linear + res    hidden -> x += . + b             [MFMA]
//   (rms_norm       x -> x, MelBandRoformer output norm)
// With fp32 weights every activation is fp32.  The residual stream stays
// fp32 in both modes, as in the reference (ops_linear.cu:167, :192).
#include <hip/hip_runtime.h>
#include <math.h>

#include <mutex>
#include <string>

#include "msst_common.hpp"

namespace msst {
namespace {

constexpr int64_t kAlign = 256;

int64_t round_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

struct StackBuffers {
    int64_t xn, big, merged, gates, tcos, tsin, fcos, fsin, total;
};

StackBuffers plan(const msst_stack_desc& d) {
    const int64_t M = d.batch * d.frames * d.bands;
    const int64_t ab = d.w_dtype == MSST_F16 ? 2 : 4;
    const int64_t hd = d.heads * d.dim_head;
    const int64_t half = d.dim_head / 2;
    StackBuffers b{};
    int64_t off = 0;
    b.xn = off; off += round_up(M * d.dim * ab);
    const int64_t big = (3 * hd > d.ff_dim ? 3 * hd : d.ff_dim);
    b.big = off; off += round_up(M * big * ab);
    b.merged = off; off += round_up(M * hd * ab);
    b.gates = off; off += round_up(M * d.heads * 4);
    b.tcos = off; off += round_up(d.frames * half * 4);
    b.tsin = off; off += round_up(d.frames * half * 4);
    b.fcos = off; off += round_up(d.bands * half * 4);
    b.fsin = off; off += round_up(d.bands * half * 4);
    b.total = off;
    return b;
}

bool desc_ok(const msst_stack_desc& d) {
    return d.batch > 0 && d.frames > 0 && d.bands > 0 && d.dim > 0 && d.heads > 0 &&
           d.dim_head == 64 && d.ff_dim > 0 && d.depth >= 0 &&
           (d.w_dtype == MSST_F16 || d.w_dtype == MSST_F32) && d.heads <= 16;
}

#define MSST_TRY(expr)              \
    do {                            \
        int rc_ = (expr);           \
        if (rc_ != MSST_OK) return rc_; \
    } while (0)

// The fused QKV + RoPE GEMM covers fp16 weights with dim % 64 == 0,
// 16-byte aligned w_qkv and fewer than 2^24 tokens.
bool rope_in_gemm(const msst_stack_desc& d, const msst_layer_weights& w) {
    const int64_t M = d.batch * d.frames * d.bands;
    const int64_t hd = d.heads * d.dim_head;
    return d.w_dtype == MSST_F16 && d.dim % 64 == 0 && (2 * hd) % 64 == 0 && M < (1 << 24) &&
           (M + 256) * d.dim * 2 < ((int64_t)1 << 31) &&
           (3 * hd + 256) * d.dim * 2 < ((int64_t)1 << 31) && aligned(w.w_qkv, 16);
}

int run_transformer(const msst_stack_desc& d, const msst_layer_weights& w, float* x, char* ws,
                    const StackBuffers& b, const msst_seq_layout& L, const float* cos_t,
                    const float* sin_t, hipStream_t s) {
    const int64_t M = d.batch * d.frames * d.bands;
    const int dt = d.w_dtype;
    const int64_t hd = d.heads * d.dim_head;
    const float nscale = sqrtf((float)d.dim);
    void* xn = ws + b.xn;
    void* qkv = ws + b.big;
    void* hidden = ws + b.big;
    void* merged = ws + b.merged;
    float* gates = reinterpret_cast<float*>(ws + b.gates);

    // Attention block (model_bs_roformer.cu:242-283) + residual (:321-322).
    MSST_TRY(msst_rms_norm_gate(x, MSST_F32, w.attn_gamma, nscale, xn, dt, w.w_gate, dt, w.b_gate,
                                gates, M, d.dim, (int)d.heads, s));
    if (rope_in_gemm(d, w)) {
        // fp16: RoPE rides in the QKV GEMM epilogue (q and k columns); the
        // attention kernel then reads pre-rotated q/k.  Position of token
        // row r: (r / tok_pos) % seq_len for both axes of either layout
        // (stack, [B,T,F]: t = (r / F) % T, f = r % F; single transformer,
        // [B,F,T]: t = r % T, f = (r / T) % F).
        MSST_TRY(msst_linear_rope(xn, w.w_qkv, nullptr, qkv, M, d.dim, 3 * hd, cos_t, sin_t,
                                  2 * hd, d.dim_head, L.tok_pos, L.seq_len, s));
        MSST_TRY(msst_gated_rope_attention(qkv, dt, 3 * hd, nullptr, nullptr, gates, merged, hd,
                                           &L, (int)d.heads, (int)d.dim_head, 0.0f, s));
    } else {
        MSST_TRY(msst_linear(xn, dt, w.w_qkv, dt, nullptr, nullptr, qkv, dt, M, d.dim, 3 * hd,
                             MSST_ACT_NONE, s));
        MSST_TRY(msst_gated_rope_attention(qkv, dt, 3 * hd, cos_t, sin_t, gates, merged, hd, &L,
                                           (int)d.heads, (int)d.dim_head, 0.0f, s));
    }
    MSST_TRY(msst_linear(merged, dt, w.w_out, dt, nullptr, x, x, MSST_F32, M, hd, d.dim,
                         MSST_ACT_NONE, s));
    // Feed-forward block (model_bs_roformer.cu:290-304) + residual (:325-326).
    MSST_TRY(msst_rms_norm(x, MSST_F32, w.ff_gamma, nscale, xn, dt, M, d.dim, s));
    MSST_TRY(msst_linear(xn, dt, w.w_ff1, dt, w.b_ff1, nullptr, hidden, dt, M, d.dim, d.ff_dim,
                         MSST_ACT_GELU, s));
    MSST_TRY(msst_linear(hidden, dt, w.w_ff2, dt, w.b_ff2, x, x, MSST_F32, M, d.ff_dim, d.dim,
                         MSST_ACT_NONE, s));
    // MelBandRoformer per-transformer output norm (model_mel_band_roformer.cu:647-648).
    if (w.final_gamma)
        MSST_TRY(msst_rms_norm(x, MSST_F32, w.final_gamma, nscale, x, MSST_F32, M, d.dim, s));
    return MSST_OK;
}

}  // namespace
}  // namespace msst

extern "C" int64_t msst_roformer_stack_workspace(const msst_stack_desc* desc) {
    using namespace msst;
    if (!desc || !desc_ok(*desc)) {
        set_error(MSST_ERR_INVALID_ARG, "msst_roformer_stack_workspace: bad descriptor");
        return -1;
    }
    return plan(*desc).total;
}

namespace msst {
namespace {

// The stack on a workspace already checked for size and alignment.
int stack_run(float* x, const msst_stack_desc& d, const msst_layer_weights* layers,
              const float* final_gamma, char* ws, const StackBuffers& b, hipStream_t s) {
    float* tcos = reinterpret_cast<float*>(ws + b.tcos);
    float* tsin = reinterpret_cast<float*>(ws + b.tsin);
    float* fcos = reinterpret_cast<float*>(ws + b.fcos);
    float* fsin = reinterpret_cast<float*>(ws + b.fsin);
    const int64_t B = d.batch, T = d.frames, F = d.bands;

    MSST_TRY(msst_rope_table_device((int)T, (int)d.dim_head, tcos, tsin, s));
    MSST_TRY(msst_rope_table_device((int)F, (int)d.dim_head, fcos, fsin, s));
    // x is worked on in place in its own [B,T,F,dim] order:
    //   time layer : sequence (b,f), position t -> token (b*T + t)*F + f
    //   freq layer : sequence (b,t), position f -> token (b*T + t)*F + f
    const msst_seq_layout time_l{B, F, T, T * F, 1, F};
    const msst_seq_layout freq_l{B * T, 1, F, F, 0, 1};
    for (int64_t i = 0; i < d.depth; ++i) {
        MSST_TRY(run_transformer(d, layers[2 * i], x, ws, b, time_l, tcos, tsin, s));
        MSST_TRY(run_transformer(d, layers[2 * i + 1], x, ws, b, freq_l, fcos, fsin, s));
    }
    // BSRoformer final norm (model_bs_roformer.cu:538-539), token-wise.
    if (final_gamma)
        MSST_TRY(msst_rms_norm(x, MSST_F32, final_gamma, sqrtf((float)d.dim), x, MSST_F32,
                               B * T * F, d.dim, s));
    return MSST_OK;
}

int check_stack_args(float* x, const msst_stack_desc* desc, const msst_layer_weights* layers) {
    MSST_REQUIRE(x && desc, MSST_ERR_INVALID_ARG, "null pointer");
    const msst_stack_desc& d = *desc;
    MSST_REQUIRE(desc_ok(d), MSST_ERR_INVALID_ARG,
                 "bad descriptor (dim_head must be 64, heads <= 16, sizes positive)");
    MSST_REQUIRE(d.depth == 0 || layers, MSST_ERR_INVALID_ARG, "null layer weights");
    for (int64_t i = 0; i < 2 * d.depth; ++i) {
        const msst_layer_weights& w = layers[i];
        MSST_REQUIRE(w.attn_gamma && w.w_qkv && w.w_gate && w.b_gate && w.w_out && w.ff_gamma &&
                         w.w_ff1 && w.b_ff1 && w.w_ff2 && w.b_ff2,
                     MSST_ERR_INVALID_ARG, "layer " + std::to_string(i) + " has a null weight");
    }
    return MSST_OK;
}

// Scratch of msst_roformer_stack_noalloc: the library's own device memory,
// one copy per GPU (each device that loads the code object holds it until
// the process ends).  Host code never passes `scratch` itself to a kernel
// or copy (on the host it only names the symbol); it uses the device
// address hipGetSymbolAddress returns, looked up once per device with that
// device current.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) char scratch[MSST_STACK_SCRATCH_BYTES];
std::mutex g_scratch_mu;
char* g_scratch_addr[kMaxDevices];

int scratch_for_current_device(char** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    MSST_REQUIRE(e == hipSuccess, MSST_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
    MSST_REQUIRE(dev >= 0 && dev < kMaxDevices, MSST_ERR_UNSUPPORTED, "device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        MSST_REQUIRE(e == hipSuccess && p, MSST_ERR_LAUNCH,
                     std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_addr[dev] = reinterpret_cast<char*>(p);
    }
    *out = g_scratch_addr[dev];
    return MSST_OK;
}

}  // namespace
}  // namespace msst

extern "C" int msst_roformer_stack(float* x, const msst_stack_desc* desc,
                                   const msst_layer_weights* layers, const float* final_gamma,
                                   void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace msst;
    MSST_TRY(check_stack_args(x, desc, layers));
    MSST_REQUIRE(workspace, MSST_ERR_INVALID_ARG, "null workspace");
    MSST_REQUIRE(aligned(workspace, kAlign), MSST_ERR_ALIGNMENT, "workspace not 256-byte aligned");
    const StackBuffers b = plan(*desc);
    MSST_REQUIRE(workspace_bytes >= b.total, MSST_ERR_WORKSPACE,
                 "workspace holds " + std::to_string(workspace_bytes) + " bytes, needs " +
                     std::to_string(b.total));
    return stack_run(x, *desc, layers, final_gamma, reinterpret_cast<char*>(workspace), b,
                     as_stream(stream));
}

extern "C" int msst_roformer_stack_noalloc(float* x, const msst_stack_desc* desc,
                                           const msst_layer_weights* layers,
                                           const float* final_gamma, void* stream) {
    using namespace msst;
    MSST_TRY(check_stack_args(x, desc, layers));
    const StackBuffers b = plan(*desc);
    MSST_REQUIRE(b.total <= MSST_STACK_SCRATCH_BYTES, MSST_ERR_WORKSPACE,
                 "the stack needs " + std::to_string(b.total) +
                     " bytes of workspace, more than the library's scratch of " +
                     std::to_string((long long)MSST_STACK_SCRATCH_BYTES) +
                     " bytes: use msst_roformer_stack with a caller workspace");
    char* ws = nullptr;
    MSST_TRY(scratch_for_current_device(&ws));
    return stack_run(x, *desc, layers, final_gamma, ws, b, as_stream(stream));
}

extern "C" int msst_roformer_stack_layer(float* x, const msst_stack_desc* desc,
                                         const msst_layer_weights* w, int axis, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && desc && w && workspace, MSST_ERR_INVALID_ARG, "null pointer");
    const msst_stack_desc& d = *desc;
    MSST_REQUIRE(desc_ok(d), MSST_ERR_INVALID_ARG,
                 "bad descriptor (dim_head must be 64, heads <= 16, sizes positive)");
    MSST_REQUIRE(axis == 0 || axis == 1, MSST_ERR_INVALID_ARG, "axis must be 0 (time) or 1 (freq)");
    MSST_REQUIRE(w->attn_gamma && w->w_qkv && w->w_gate && w->b_gate && w->w_out && w->ff_gamma &&
                     w->w_ff1 && w->b_ff1 && w->w_ff2 && w->b_ff2,
                 MSST_ERR_INVALID_ARG, "null weight");
    MSST_REQUIRE(aligned(workspace, kAlign), MSST_ERR_ALIGNMENT, "workspace not 256-byte aligned");
    const StackBuffers b = plan(d);
    MSST_REQUIRE(workspace_bytes >= b.total, MSST_ERR_WORKSPACE,
                 "workspace holds " + std::to_string(workspace_bytes) + " bytes, needs " +
                     std::to_string(b.total));
    hipStream_t s = as_stream(stream);
    char* ws = reinterpret_cast<char*>(workspace);
    const int64_t B = d.batch, T = d.frames, F = d.bands;
    float* cs = reinterpret_cast<float*>(ws + (axis == 0 ? b.tcos : b.fcos));
    float* sn = reinterpret_cast<float*>(ws + (axis == 0 ? b.tsin : b.fsin));
    MSST_TRY(msst_rope_table_device((int)(axis == 0 ? T : F), (int)d.dim_head, cs, sn, s));
    // The stack's own [B,T,F,dim] addressing (stack_run).
    const msst_seq_layout time_l{B, F, T, T * F, 1, F};
    const msst_seq_layout freq_l{B * T, 1, F, F, 0, 1};
    return run_transformer(d, *w, x, ws, b, axis == 0 ? time_l : freq_l, cs, sn, s);
}

extern "C" int msst_roformer_transformer(float* x, const msst_stack_desc* desc,
                                         const msst_layer_weights* w, int axis, void* workspace,
                                         int64_t workspace_bytes, void* stream) {
    using namespace msst;
    MSST_REQUIRE(x && desc && w && workspace, MSST_ERR_INVALID_ARG, "null pointer");
    const msst_stack_desc& d = *desc;
    MSST_REQUIRE(desc_ok(d), MSST_ERR_INVALID_ARG,
                 "bad descriptor (dim_head must be 64, heads <= 16, sizes positive)");
    MSST_REQUIRE(axis == 0 || axis == 1, MSST_ERR_INVALID_ARG, "axis must be 0 (time) or 1 (freq)");
    MSST_REQUIRE(w->attn_gamma && w->w_qkv && w->w_gate && w->b_gate && w->w_out && w->ff_gamma &&
                     w->w_ff1 && w->b_ff1 && w->w_ff2 && w->b_ff2,
                 MSST_ERR_INVALID_ARG, "null weight");
    MSST_REQUIRE(aligned(workspace, kAlign), MSST_ERR_ALIGNMENT, "workspace not 256-byte aligned");
    const StackBuffers b = plan(d);
    MSST_REQUIRE(workspace_bytes >= b.total, MSST_ERR_WORKSPACE,
                 "workspace holds " + std::to_string(workspace_bytes) + " bytes, needs " +
                     std::to_string(b.total));
    hipStream_t s = as_stream(stream);
    char* ws = reinterpret_cast<char*>(workspace);
    const int64_t B = d.batch, T = d.frames, F = d.bands;
    float* cs = reinterpret_cast<float*>(ws + (axis == 0 ? b.tcos : b.fcos));
    float* sn = reinterpret_cast<float*>(ws + (axis == 0 ? b.tsin : b.fsin));
    MSST_TRY(msst_rope_table_device((int)(axis == 0 ? T : F), (int)d.dim_head, cs, sn, s));
    const msst_seq_layout time_l{B * F, 1, T, T, 0, 1};
    const msst_seq_layout freq_l{B, T, F, F * T, 1, T};
    return run_transformer(d, *w, x, ws, b, axis == 0 ? time_l : freq_l, cs, sn, s);
}
