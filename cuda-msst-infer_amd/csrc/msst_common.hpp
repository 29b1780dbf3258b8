// msst_common.hpp — shared device types, MFMA wrappers, epilogue math and
// the host-side status plumbing of the C ABI (include/msst_hip.h).
//
// Target: gfx950 only (wave64, v_mfma_f32_{32x32x16,16x16x32}_f16,
// v_mfma_f32_{32x32x2,16x16x4}_f32, 160 KB LDS per CU).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "msst_hip.h"

namespace msst {

typedef _Float16 half_t;
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4v __attribute__((ext_vector_type(4)));
typedef unsigned int u2v __attribute__((ext_vector_type(2)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));
typedef unsigned int u2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// MFMA wrappers.  Lane layouts (l = lane, h = l / 32 for 32-wide shapes):
//   32x32x16 f16:  A lane holds A[l%32][8h .. 8h+7]; B lane holds
//                  B[8h .. 8h+7][l%32]; D register v holds
//                  D[8*(v/4) + 4h + v%4][l%32].
//   32x32x2 f32:   A lane holds A[l%32][h]; B lane holds B[h][l%32];
//                  D as above.
// The K index handed to a lane only has to agree between A and B, so the
// kernels map K positions to (lane half, register) however suits their LDS
// layout.
// ---------------------------------------------------------------------------
__device__ __forceinline__ f16x mfma32x32x16(h8 a, h8 b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x mfma32x32x2f32(float a, float b, f16x c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Epilogue activations.
// GELU(v) = v Phi(v), Phi(v) = (1 + erf(v / sqrt 2)) / 2, the reference's
// 0.5 v (1 + erff(v / sqrt 2)) (ops_fused.cu:21-24).  With a = |v| and
// c = Phi(-a), v Phi(v) is v (1 - c) for v >= 0 and v c for v < 0: both are
// v / 2 + a (1/2 - c), one FMA with |v| as a free source modifier instead of
// a select on the sign.  c = 2^P(x), x = min(a, 5.6) (v_minimum_f32, which
// does not canonicalise its operands as fminf would), P of degree 6: log2 Phi(-x) fitted minimax in
// the absolute error of c on [0, 5.6] (a linear program on 3000 points,
// gelu_fit.py beside this file regenerates the coefficients), |error of c|
// <= 8.9e-8.  Past 5.6 the clamp keeps c = Phi(-5.6) = 1.1e-8, which rounds
// away against 1/2.  Eleven VALU operations with one v_exp_f32, against
// thirteen with v_exp_f32 and v_rcp_f32 for the rational erf of Abramowitz &
// Stegun 7.1.26 (FF1 168 -> 162 us) and several times that for the library
// erff.  Error, with fp32 evaluation and v_exp_f32 off by one ulp either
// way: <= 2.4e-7 |v| over all finite v, far below the fp16 output rounding
// and the 1e-4 fp32 tolerance.  v = +inf gives +inf, v = -inf NaN (as
// 0.5 v (1 + erf) does), NaN stays NaN.
// sigmoid(v) = 1 / (1 + 2^(-v log2 e)) with v_exp_f32 and v_rcp_f32 (each
// about 1 ulp): relative error ~3e-7 in 4 VALU operations instead of the
// library expf and an IEEE division; v -> -inf gives rcp(inf) = 0, v -> +inf
// gives 1.  SiLU = v sigmoid(v).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float gelu_erf(float v) {
    const float a = fabsf(v);
    // v_minimum_f32: no canonicalisation, and a NaN stays NaN.
    const float x = __builtin_elementwise_minimum(a, 5.6f);
    float p = fmaf(x, 1.984903428819962e-05f, -6.632566801272333e-04f);
    p = fmaf(x, p, 7.766014896333218e-03f);
    p = fmaf(x, p, -5.297756940126419e-02f);
    p = fmaf(x, p, -4.590558707714081e-01f);
    p = fmaf(x, p, -1.151121973991394f);
    p = fmaf(x, p, -9.999997615814209e-01f);
    const float c = __builtin_amdgcn_exp2f(p);
    return fmaf(a, 0.5f - c, 0.5f * v);
}

__device__ __forceinline__ float sigmoid_fast(float v) {
    return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(v * -1.4426950408889634f));
}

// tanh(x) = (e^2x - 1) / (e^2x + 1) with e^2x from v_exp_f32 (|x| clamped to
// 9, where tanh rounds to +-1 in fp32), and the odd Taylor polynomial
// x - x^3/3 + 2x^5/15 for |x| < 1/16 (truncation <= 17 x^7 / 315, a relative
// 3e-9 at 1/16), where the quotient would lose digits to e^2x - 1.
// Absolute error ~2e-7 (a few fp32 ulps of 1); six VALU operations on the
// main branch against several times that for the library tanhf.
__device__ __forceinline__ float tanh_fast(float x) {
    const float xc = fminf(fmaxf(x, -9.0f), 9.0f);
    const float t = __builtin_amdgcn_exp2f(xc * 2.8853900817779268f);  // e^(2x)
    const float q = (t - 1.0f) * __builtin_amdgcn_rcpf(t + 1.0f);
    const float x2 = x * x;
    const float p = x * fmaf(x2, fmaf(x2, 0.13333333333333333f, -0.33333333333333333f), 1.0f);
    return fabsf(x) < 0.0625f ? p : q;
}

// Compile-time activation (ACT = MSST_ACT_*), and the runtime form for
// kernels that take it as an argument.
template <int ACT>
__device__ __forceinline__ float act_fixed(float v) {
    if constexpr (ACT == MSST_ACT_GELU)
        return gelu_erf(v);
    else if constexpr (ACT == MSST_ACT_SIGMOID)
        return sigmoid_fast(v);
    else if constexpr (ACT == MSST_ACT_SILU)
        return v * sigmoid_fast(v);
    else
        return v;
}

__device__ __forceinline__ float act_apply(float v, int act) {
    if (act == MSST_ACT_GELU) return act_fixed<MSST_ACT_GELU>(v);
    if (act == MSST_ACT_SIGMOID) return act_fixed<MSST_ACT_SIGMOID>(v);
    if (act == MSST_ACT_SILU) return act_fixed<MSST_ACT_SILU>(v);
    return v;
}

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

template <typename T>
__device__ __forceinline__ T from_f32(float v) { return (T)v; }

// ---------------------------------------------------------------------------
// LDS DMA (buffer_load_dwordx4 ... lds): lane l's 16 bytes at buffer offset
// voffset land at lds + 16 * l (lds is wave-uniform).  Offsets at or past
// `bytes` read zero.  The buffer descriptor type only exists in device code,
// so kernels reach it through this helper (a kernel naming it loses its
// host stub).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ void dma16(const void* base, int bytes, half_t* lds, uint32_t voffset) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds, 16, voffset, 0, 0, 0);
}

// LDS-typed (address space 3) pointers: 32-bit LDS addresses, so address
// arithmetic folds into ds_* immediates instead of per-access conversions
// from generic pointers.
typedef __attribute__((address_space(3))) half_t lds_half_t;
typedef __attribute__((address_space(3))) h8 lds_h8_t;

__device__ __forceinline__ void dma16(const void* base, int bytes, lds_half_t* lds,
                                      uint32_t voffset) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds, 16, voffset, 0, 0, 0);
}

// 16 bytes at byte offset off of [base, base + bytes); zeros past the end.
__device__ __forceinline__ f4 load16_bounded(const float* base, int bytes, uint32_t off) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, bytes, 0x00020000);
    return __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
}

// Makes the compiler complete whatever produces v (a load: its s_waitcnt)
// at this point of the program, with no instruction of its own.
__device__ __forceinline__ void use_now(const f16x& v) { asm volatile("" ::"v"(v)); }

// A pointer the compiler can keep in SGPRs (the value is wave-uniform by
// construction; without this, a buffer descriptor built from it is
// waterfalled, one loop iteration per distinct lane value).
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() carries a
// workgroup release/acquire fence, which the compiler lowers to
// s_waitcnt vmcnt(0) before s_barrier: it waits for every outstanding
// global load, store and LDS DMA of the wave, including DMAs issued for
// later ring stages and stores that nothing reads back.  Callers of this
// barrier wait for exactly what the other waves need (their own
// s_waitcnt vmcnt(N) for DMA stages); LDS reads/writes are drained here.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// q = n / d, r = n % d for 0 <= n < 2^24, d >= 1, inv_d = 1.0f / d: the
// float quotient is within one of the true one (relative error <= 2^-23,
// n / d < 2^24 / d), and one correction step makes it exact.
__device__ __forceinline__ int divmod24(int n, int d, float inv_d, int& r) {
    int q = (int)((float)n * inv_d);
    r = n - q * d;
    if (r < 0) {
        --q;
        r += d;
    } else if (r >= d) {
        ++q;
        r -= d;
    }
    return q;
}

// Butterfly sum over the 64 lanes of a wave.
// Sum over the 64 lanes with DPP lane moves (no LDS round trips): butterfly
// within quads, mirrors within 8- and 16-lane rows, then the row broadcasts
// carry rows 0-2 into lane 63, which is read back as a wave-uniform value.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_move(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ float dpp_wave_sum(float v) {
    v += dpp_move<0xB1, 0xF>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E, 0xF>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x141, 0xF>(v);  // row_half_mirror
    v += dpp_move<0x140, 0xF>(v);  // row_mirror
    v += dpp_move<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_move<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Eight per-lane partial sums (one per gate) reduced over the wave, with the
// sum of gate g left in the eight lanes 8g .. 8g + 7.  Each step halves the
// values a lane carries: the xor-32 and xor-16 exchanges pair two registers
// through v_permlane32_swap / v_permlane16_swap (no selects needed), the
// xor-8 one picks by lane bit 3 and moves by DPP row_ror:8; the last three
// lane bits are summed with DPP (quad perms, row_half_mirror).  21 VALU
// operations against 8 full wave sums.
__device__ __forceinline__ float gate_sums8(const float (&v)[8], int lane) {
    float c[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // lane bit 5: values i (clear) / i + 4 (set)
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]),
                                                        false, false);
        c[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    float d[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // lane bit 4: + 0 / + 2
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(c[i]), __float_as_uint(c[i + 2]),
                                                        false, false);
        d[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = (lane & 8) != 0;  // lane bit 3: + 0 / + 1
    const float keep = b3 ? d[1] : d[0];
    const float send = b3 ? d[0] : d[1];
    float s = keep + dpp_move<0x128, 0xF>(send);  // row_ror:8 = lane ^ 8 within a row
    s += dpp_move<0xB1, 0xF>(s);   // quad_perm [1,0,3,2]
    s += dpp_move<0x4E, 0xF>(s);   // quad_perm [2,3,0,1]
    s += dpp_move<0x141, 0xF>(s);  // row_half_mirror
    return s;
}

// Sum over the wave, the same value in every lane (all 64 lanes active).
__device__ __forceinline__ float wave_sum(float v) { return dpp_wave_sum(v); }

// ---------------------------------------------------------------------------
// Host-side status helpers.
// ---------------------------------------------------------------------------
int set_error(int code, const std::string& msg);
int check_launch(const char* what);

inline bool is_dtype(int dt) { return dt == MSST_F32 || dt == MSST_F16; }
inline size_t dtype_bytes(int dt) { return dt == MSST_F16 ? 2 : 4; }
inline bool aligned(const void* p, size_t a) {
    return (reinterpret_cast<uintptr_t>(p) % a) == 0;
}
inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

}  // namespace msst

#define MSST_REQUIRE(cond, code, msg)                                   \
    do {                                                                \
        if (!(cond)) return ::msst::set_error((code), std::string(__func__) + ": " + (msg)); \
    } while (0)
