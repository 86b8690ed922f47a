// Shared device helpers for the gfx950 kernels: bf16 conversion, vector
// types, wavefront (64-lane) reductions, and the GELU used by the GEGLU and
// scorer epilogues.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

typedef uint16_t bf16_t;  // bf16 bit pattern in memory
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

#define JH_WAVE 64

// Error raised by host code; the C-ABI layer turns it into a return code.
struct jh_error : std::runtime_error {
    int code;
    jh_error(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

#define HIP_CHECK(call)                                                                              \
    do {                                                                                             \
        hipError_t e_ = (call);                                                                      \
        if (e_ != hipSuccess)                                                                        \
            throw jh_error(2, std::string(#call) + ": " + hipGetErrorString(e_));                    \
    } while (0)

// float -> bf16 bits on the host, round to nearest even, NaN kept quiet
// (as half::bf16::from_f32, used for the one-time weight conversion).
inline bf16_t f2bf_host(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (bf16_t)(u >> 16);
}

// Device conversions use gfx950's v_cvt_pk_bf16_f32 (round to nearest even).
__device__ inline bf16_t f2bf(float f) { return __builtin_bit_cast(bf16_t, (__bf16)f); }

__host__ __device__ inline float bf2f(bf16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Two floats -> packed bf16x2 (low half = a), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// Raw buffer resource (stride 0, 32-bit data format) over [base, base + bytes),
// for buffer_load ... lds operand DMA.
__device__ inline i32x4 make_rsrc(const void* base, uint64_t bytes) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    return i32x4{(int)(uint32_t)p, (int)(uint32_t)(p >> 32),
                 (int)(uint32_t)(bytes < 0xffffffffull ? bytes : 0xffffffffull), 0x00020000};
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, JH_WAVE);
    return v;
}
// wave_sum of N values at once (the same steps for each), so their shuffles
// share each LDS round trip.
template <int N>
__device__ inline void wave_sum_n(float (&v)[N]) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
#pragma unroll
        for (int r = 0; r < N; ++r) v[r] += __shfl_xor(v[r], o, JH_WAVE);
}

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, JH_WAVE));
    return v;
}

// erf by the rational approximation published in Eigen (ptanh/perf float
// coefficients, as used by XLA): clamp to [-4, 4], x·P(x²)/Q(x²), |error| < 1e-6.
// The quotient uses the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an
// IEEE division (~10 instructions): the difference, below 2^-22 relative, is
// far under the approximation's own error and the bf16 rounding of GEGLU.
__device__ inline float erf_rational(float x) {
#pragma clang fp contract(off)
    x = fminf(fmaxf(x, -4.0f), 4.0f);
    const float x2 = x * x;
    float p = -2.72614225801306e-10f;
    p = __builtin_fmaf(p, x2, 2.77068142495902e-08f);
    p = __builtin_fmaf(p, x2, -2.10102402082508e-06f);
    p = __builtin_fmaf(p, x2, -5.69250639462346e-05f);
    p = __builtin_fmaf(p, x2, -7.34990630326855e-04f);
    p = __builtin_fmaf(p, x2, -2.95459980854025e-03f);
    p = __builtin_fmaf(p, x2, -1.60960333262415e-02f);
    float q = -1.45660718464996e-05f;
    q = __builtin_fmaf(q, x2, -2.13374055278905e-04f);
    q = __builtin_fmaf(q, x2, -1.68282697438203e-03f);
    q = __builtin_fmaf(q, x2, -7.37332916720468e-03f);
    q = __builtin_fmaf(q, x2, -1.42647390514189e-02f);
    return x * p * __builtin_amdgcn_rcpf(q);
}

// Exact-form GELU 0.5·x·(1 + erf(x/√2)), as nn.GELU() / transformers "gelu".
// Its operations (and erf_rational's) are written out with contraction off, so
// every inlined copy rounds the same way: an output element is a function of
// its input alone, whichever kernel or epilogue site computes it.
__device__ inline float gelu_erf(float x) {
#pragma clang fp contract(off)
    return 0.5f * x * (1.0f + erf_rational(x * 0.70710678118654752f));
}

// Rotate-half RoPE of one (d, d + 32) pair: lo' = lo·c − hi·s, hi' = hi·c + lo·s,
// each as one rounded product and one fused multiply-add.  Spelling the FMAs
// out fixes the rounding sequence, so every kernel and every inlined copy (the
// GEMM epilogues run it at several sites) gives the same bits for a token.
__device__ inline void rope_rotate(float& lo, float& hi, float c, float s) {
    const float x0 = lo, x1 = hi;
    lo = __builtin_fmaf(x0, c, -(x1 * s));
    hi = __builtin_fmaf(x1, c, x0 * s);
}
