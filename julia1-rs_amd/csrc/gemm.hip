// BF16 x BF16 -> FP32 MFMA GEMM for gfx950 with fused epilogues.
//
// out = epi(X · Wᵀ): X [rows, K] bf16 (optionally row-gathered), W [N, K] bf16
// (PyTorch Linear layout).  Both operands are K-contiguous, so both stream
// into LDS as plain 16-byte row chunks.  The MFMA "M" dimension is the output
// feature and "N" the token: v_mfma_f32_32x32x16_bf16 then leaves each lane
// holding, for one token, four runs of four consecutive features — which is
// what the epilogues want: 16-byte FP32 residual read-modify-writes, and the
// RoPE pair (d, d+32) and the GEGLU pair (gate, up) in the same lane.
//
// Workgroup tile BF features x BT tokens x BK=64, LDS double-buffered with
// register prefetch (one barrier per K step).  LDS rows are padded to 72
// bf16 (144 B) so the 16-byte fragment reads of 8 consecutive rows hit
// distinct banks.  Tiles are assigned XCD-contiguously: MI355X deals
// workgroups round-robin to its 8 XCDs, so tile t is given to workgroup
// b with b % 8 = XCD, keeping each XCD's L2 on a contiguous band of tokens.
#include <hip/hip_runtime.h>

#include "../../include/julia1_hip_ops.h"
#include "kernels.hpp"

namespace {

constexpr int BK = 64;
constexpr int LDS_STRIDE = 72;

template <int EPI, int BF, int BT, int WF, int WT>
__global__ __launch_bounds__(WF* WT * 64) void gemm_kernel(GemmArgs a) {
    constexpr int NT = WF * WT * 64;
    constexpr int FPW = BF / WF, TPW = BT / WT;  // features / tokens per wave
    constexpr int FB = FPW / 32, TB = TPW / 32;  // 32x32 MFMA blocks per wave
    constexpr int CW = BF * 8 / NT, CX = BT * 8 / NT;  // 16-byte chunks per thread per K step
    static_assert(CW * NT == BF * 8 && CX * NT == BT * 8, "tile must split evenly over threads");
    static_assert(FB >= 1 && TB >= 1, "wave tile too small");
    static_assert((EPI != JH_EPI_ROPE_BF16 && EPI != JH_EPI_GEGLU_BF16) || FB % 2 == 0,
                  "pair epilogues need 64-feature wave slabs");

    __shared__ __align__(16) bf16_t sW[2][BF][LDS_STRIDE];
    __shared__ __align__(16) bf16_t sX[2][BT][LDS_STRIDE];

    const int tid = threadIdx.x;
    const int nF = (a.n + BF - 1) / BF;
    const int nTk = (a.rows + BT - 1) / BT;
    const int ntiles = nF * nTk;
    const int b = blockIdx.x;
    const int xcd = b & 7, local = b >> 3, q8 = ntiles >> 3, r8 = ntiles & 7;
    const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    const int f0 = (tile % nF) * BF, t0 = (tile / nF) * BT;

    // Per-thread source rows for the global->LDS copies (fixed across K steps).
    const bf16_t* wsrc[CW];
    const bf16_t* xsrc[CX];
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        int c = tid + NT * i, row = c >> 3, kc = c & 7;
        int f = f0 + row;
        wsrc[i] = f < a.n ? a.w + (long)f * a.k + kc * 8 : nullptr;
    }
#pragma unroll
    for (int i = 0; i < CX; ++i) {
        int c = tid + NT * i, row = c >> 3, kc = c & 7;
        int t = t0 + row;
        if (t < a.rows) {
            long src = a.gather ? (long)a.gather[t] : (long)t;
            xsrc[i] = a.x + src * a.ldx + kc * 8;
        } else {
            xsrc[i] = nullptr;
        }
    }

    u32x4 rw[CW], rx[CX];
    auto gload = [&](int kt) {
        const int kb = kt * BK;
#pragma unroll
        for (int i = 0; i < CW; ++i) rw[i] = wsrc[i] ? *(const u32x4*)(wsrc[i] + kb) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < CX; ++i) rx[i] = xsrc[i] ? *(const u32x4*)(xsrc[i] + kb) : u32x4{0, 0, 0, 0};
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < CW; ++i) {
            int c = tid + NT * i;
            *(u32x4*)&sW[buf][c >> 3][(c & 7) * 8] = rw[i];
        }
#pragma unroll
        for (int i = 0; i < CX; ++i) {
            int c = tid + NT * i;
            *(u32x4*)&sX[buf][c >> 3][(c & 7) * 8] = rx[i];
        }
    };

    const int lane = tid & 63, wave = tid >> 6;
    const int wf = wave % WF, wt = wave / WF;
    const int lr = lane & 31, lk = (lane >> 5) * 8;

    f32x16 acc[FB][TB];
#pragma unroll
    for (int i = 0; i < FB; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    const int KT = a.k / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8 af[FB], bx[TB];
#pragma unroll
            for (int i = 0; i < FB; ++i) af[i] = *(const bf16x8*)&sW[buf][wf * FPW + i * 32 + lr][ks * 16 + lk];
#pragma unroll
            for (int j = 0; j < TB; ++j) bx[j] = *(const bf16x8*)&sX[buf][wt * TPW + j * 32 + lr][ks * 16 + lk];
#pragma unroll
            for (int i = 0; i < FB; ++i)
#pragma unroll
                for (int j = 0; j < TB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bx[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) sstore(buf ^ 1);
        __syncthreads();
    }

    // Epilogue.  acc[i][j][e]: feature fslab(i) + (e/4)*8 + g4 + e%4, token t(j).
    const int g4 = (lane >> 5) * 4;
#pragma unroll
    for (int j = 0; j < TB; ++j) {
        const int t = t0 + wt * TPW + j * 32 + lr;
        if (t >= a.rows) continue;
        if constexpr (EPI == JH_EPI_ROPE_BF16 || EPI == JH_EPI_GEGLU_BF16) {
#pragma unroll
            for (int i = 0; i < FB; i += 2) {
                const int slab = f0 + wf * FPW + i * 32;  // 64-aligned: [slab, slab+32) pairs with [slab+32, slab+64)
                if (slab >= a.n) continue;
                if constexpr (EPI == JH_EPI_ROPE_BF16) {
                    bf16_t* o = (bf16_t*)a.out + (long)t * a.ldo + a.col + slab;
                    const bool rot = slab < a.rope_cols;
                    const long p = rot ? (long)(a.pos[t] & 0xffff) * 32 : 0;
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const int d = qd * 8 + g4;
                        float lo[4], hi[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            lo[e] = acc[i][j][qd * 4 + e];
                            hi[e] = acc[i + 1][j][qd * 4 + e];
                        }
                        if (rot) {
                            f32x4 c = *(const f32x4*)(a.cos_t + p + d);
                            f32x4 s = *(const f32x4*)(a.sin_t + p + d);
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                float x0 = lo[e], x1 = hi[e];
                                lo[e] = x0 * c[e] - x1 * s[e];
                                hi[e] = x1 * c[e] + x0 * s[e];
                            }
                        }
                        *(u32x2*)(o + d) = u32x2{pack2(lo[0], lo[1]), pack2(lo[2], lo[3])};
                        *(u32x2*)(o + 32 + d) = u32x2{pack2(hi[0], hi[1]), pack2(hi[2], hi[3])};
                    }
                } else {
                    bf16_t* o = (bf16_t*)a.out + (long)t * a.ldo + a.col + slab / 2;
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        const int d = qd * 8 + g4;
                        float g[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) g[e] = gelu_erf(acc[i][j][qd * 4 + e]) * acc[i + 1][j][qd * 4 + e];
                        *(u32x2*)(o + d) = u32x2{pack2(g[0], g[1]), pack2(g[2], g[3])};
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < FB; ++i) {
                const int slab = f0 + wf * FPW + i * 32;
                if (slab >= a.n) continue;
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int f = slab + qd * 8 + g4;
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][qd * 4 + e];
                    if constexpr (EPI == JH_EPI_STORE_BF16) {
                        bf16_t* o = (bf16_t*)a.out + (long)t * a.ldo + a.col + f;
                        *(u32x2*)o = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
                    } else if constexpr (EPI == JH_EPI_RESID_F32) {
                        float* o = (float*)a.out + (long)t * a.ldo + a.col + f;
                        f32x4 old = *(const f32x4*)o;
                        if (a.bias) {
                            f32x4 bb = *(const f32x4*)(a.bias + f);
#pragma unroll
                            for (int e = 0; e < 4; ++e) old[e] += v[e] + bb[e];
                        } else {
#pragma unroll
                            for (int e = 0; e < 4; ++e) old[e] += v[e];
                        }
                        *(f32x4*)o = old;
                    } else {
                        f32x4 bb = *(const f32x4*)(a.bias + f);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[e] += bb[e];
                            if constexpr (EPI == JH_EPI_BIAS_RELU_BF16) v[e] = fmaxf(v[e], 0.0f);
                        }
                        if constexpr (EPI == JH_EPI_BIAS_F32) {
                            *(f32x4*)((float*)a.out + (long)t * a.ldo + a.col + f) = f32x4{v[0], v[1], v[2], v[3]};
                        } else {
                            bf16_t* o = (bf16_t*)a.out + (long)t * a.ldo + a.col + f;
                            *(u32x2*)o = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
                        }
                    }
                }
            }
        }
    }
}

template <int EPI>
void launch_cfg(const GemmArgs& a, hipStream_t s) {
    constexpr int BF = 128, BT = 128, WF = 2, WT = 2;
    int nF = (a.n + BF - 1) / BF, nTk = (a.rows + BT - 1) / BT;
    int blocks = nF * nTk;
    hipLaunchKernelGGL((gemm_kernel<EPI, BF, BT, WF, WT>), dim3(blocks), dim3(WF * WT * 64), 0, s, a);
    HIP_CHECK(hipGetLastError());
}

}  // namespace

void launch_gemm(int epi, const GemmArgs& a, hipStream_t s) {
    if (a.rows < 0 || a.n <= 0 || a.k <= 0 || a.k % BK || a.n % 64 || a.k > 8192)
        throw jh_error(1, "gemm: need K % 64 == 0, N % 64 == 0, K <= 8192");
    if (a.rows == 0) return;
    if (!a.x || !a.w || !a.out) throw jh_error(1, "gemm: null operand");
    if (a.ldx % 8 || a.ldx < a.k || ((uintptr_t)a.x & 15) || ((uintptr_t)a.w & 15))
        throw jh_error(1, "gemm: x/w must be 16-byte aligned with ldx % 8 == 0 and ldx >= K");
    const bool f32out = epi == JH_EPI_RESID_F32 || epi == JH_EPI_BIAS_F32;
    const long width = epi == JH_EPI_GEGLU_BF16 ? a.n / 2 : a.n;
    if (a.col < 0 || a.ldo < a.col + width || a.ldo % 4 || a.col % 4 || ((uintptr_t)a.out & (f32out ? 15 : 7)))
        throw jh_error(1, "gemm: output columns out of range or misaligned");
    const bool needs_bias = epi == JH_EPI_BIAS_BF16 || epi == JH_EPI_BIAS_RELU_BF16 || epi == JH_EPI_BIAS_F32;
    if (needs_bias && !a.bias) throw jh_error(1, "gemm: epilogue needs a bias");
    if (epi == JH_EPI_ROPE_BF16 && a.rope_cols > 0 && (!a.pos || !a.cos_t || !a.sin_t || a.rope_cols % 64))
        throw jh_error(1, "gemm: RoPE epilogue needs pos, cos, sin and rope_cols % 64 == 0");
    if (epi == JH_EPI_GEGLU_BF16 && a.n % 64) throw jh_error(1, "gemm: GEGLU needs N % 64 == 0");
    switch (epi) {
        case JH_EPI_STORE_BF16: launch_cfg<JH_EPI_STORE_BF16>(a, s); break;
        case JH_EPI_ROPE_BF16: launch_cfg<JH_EPI_ROPE_BF16>(a, s); break;
        case JH_EPI_GEGLU_BF16: launch_cfg<JH_EPI_GEGLU_BF16>(a, s); break;
        case JH_EPI_RESID_F32: launch_cfg<JH_EPI_RESID_F32>(a, s); break;
        case JH_EPI_BIAS_BF16: launch_cfg<JH_EPI_BIAS_BF16>(a, s); break;
        case JH_EPI_BIAS_RELU_BF16: launch_cfg<JH_EPI_BIAS_RELU_BF16>(a, s); break;
        case JH_EPI_BIAS_F32: launch_cfg<JH_EPI_BIAS_F32>(a, s); break;
        default: throw jh_error(1, "gemm: unknown epilogue");
    }
}
