// One row of `hidden` = 64*EPL floats spread over a 64-lane wavefront,
// hidden/64 values per lane, loaded with the widest vector that divides them
// (float4 for hidden 768/1024, float2 for 384/128), so every global access is
// a fully coalesced 64-lane vector load; and the two-pass LayerNorm over it
// (mean, then squared deviations, with wavefront-shuffle sums).  Shared by the
// row kernels and the small-batch GEMM's LayerNorm prologue, so both produce
// the same bits.
#pragma once

#include "common.hpp"

template <int EPL>
struct RowVec {
    static constexpr int VEC = EPL % 4 == 0 ? 4 : (EPL % 2 == 0 ? 2 : 1);
    static constexpr int NC = EPL / VEC;  // vector chunks per lane
    float v[EPL];

    // Chunk c of this lane covers elements [(c*64 + lane)*VEC, +VEC).
    __device__ static int index(int c, int lane) { return (c * 64 + lane) * VEC; }

    __device__ void load(const float* row, int lane) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float* p = row + index(c, lane);
            if constexpr (VEC == 4) {
                f32x4 t = *(const f32x4*)p;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[c * 4 + e] = t[e];
            } else if constexpr (VEC == 2) {
                float2 t = *(const float2*)p;
                v[c * 2] = t.x;
                v[c * 2 + 1] = t.y;
            } else {
                v[c] = *p;
            }
        }
    }
    __device__ void store(float* row, int lane) const {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            float* p = row + index(c, lane);
            if constexpr (VEC == 4) {
                *(f32x4*)p = f32x4{v[c * 4], v[c * 4 + 1], v[c * 4 + 2], v[c * 4 + 3]};
            } else if constexpr (VEC == 2) {
                *(float2*)p = make_float2(v[c * 2], v[c * 2 + 1]);
            } else {
                *p = v[c];
            }
        }
    }
    __device__ void store_bf16(bf16_t* row, int lane) const {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            bf16_t* p = row + index(c, lane);
            if constexpr (VEC == 4) {
                *(u32x2*)p = u32x2{pack2(v[c * 4], v[c * 4 + 1]), pack2(v[c * 4 + 2], v[c * 4 + 3])};
            } else if constexpr (VEC == 2) {
                *(uint32_t*)p = pack2(v[c * 2], v[c * 2 + 1]);
            } else {
                *p = f2bf(v[c]);
            }
        }
    }
    // v = (v - mean) * rstd * w (+ b), two-pass statistics over the whole row.
    // (The bias branch names &bb only where it is loaded: a pointer that may
    // point at a local or be null keeps that local in scratch memory.)
    __device__ void layer_norm(const float* w, const float* b, float eps, int lane) {
        RowVec<EPL> g;
        g.load(w, lane);
        if (b) {
            RowVec<EPL> bb;
            bb.load(b, lane);
            layer_norm(g, &bb, eps);
        } else {
            layer_norm(g, nullptr, eps);
        }
    }
    // The same with the weights (and the bias, when bb is non-null) already
    // loaded, in the steps below.
    __device__ void layer_norm(const RowVec<EPL>& g, const RowVec<EPL>* bb, float eps) {
        const float mean = wave_sum(sum()) * kInvN;
        scale_shift(mean, rstd(wave_sum(sq_dev(mean)), eps), g, bb);
    }
    // Steps of layer_norm, for callers that reduce several rows together.
    static constexpr float kInvN = 1.0f / (EPL * 64);
    __device__ float sum() const {
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) s += v[e];
        return s;
    }
    // The multiply-adds are explicit FMAs: left to the compiler, contraction
    // can be decided per inlined instance, and one row of the GEMM prologue
    // once rounded differently from layer_norm_kernel on the same values.
    __device__ static float rstd(float sq_sum, float eps) {
        return 1.0f / __builtin_sqrtf(__builtin_fmaf(sq_sum, kInvN, eps));
    }
    __device__ float sq_dev(float mean) const {
        float q = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float d = v[e] - mean;
            q = __builtin_fmaf(d, d, q);
        }
        return q;
    }
    __device__ void scale_shift(float mean, float rs, const RowVec<EPL>& g, const RowVec<EPL>* bb) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float t = (v[e] - mean) * rs;
            v[e] = bb ? __builtin_fmaf(t, g.v[e], bb->v[e]) : t * g.v[e];
        }
    }
};
