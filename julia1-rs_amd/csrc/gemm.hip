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
// Pipeline: workgroup tile BF features x BT tokens x BK=64.  Global loads run
// two K steps ahead of the MFMAs (two register stages), LDS is double
// buffered, one barrier per K step.  At K = 768 that keeps 2/12 of the whole
// operand stream in flight per workgroup, which hides the HBM/MALL latency.
// All loads are unconditional (out-of-range rows are clamped) so the
// compiler's vmcnt waits stay exact.  LDS rows are padded to 72 bf16 (144 B)
// so the 16-byte fragment reads of 8 consecutive rows hit distinct banks.
//
// Tiles are dealt XCD-contiguously: MI355X hands workgroups round-robin to its
// 8 XCDs, so tile t goes to the workgroup whose id mod 8 selects the XCD that
// owns t's band; inside a band, tiles are grouped 8 token blocks at a time so
// the operands resident on one XCD fit its 4 MB L2.
#include <hip/hip_runtime.h>

#include "../../include/julia1_hip_ops.h"
#include "kernels.hpp"

namespace {

constexpr int BK = 64;
constexpr int LDS_STRIDE = 72;

template <int EPI, int FB, int TB>
__device__ inline void epilogue(const GemmArgs& a, f32x16 (&acc)[FB][TB], int fw0, int tw0, int lane) {
    // acc[i][j][e]: feature fw0 + i*32 + (e/4)*8 + g4 + e%4, token tw0 + j*32 + lr.
    const int g4 = (lane >> 5) * 4, lr = lane & 31;
#pragma unroll
    for (int j = 0; j < TB; ++j) {
        const int t = tw0 + j * 32 + lr;
        if (t >= a.rows) continue;
        if constexpr (EPI == JH_EPI_ROPE_BF16 || EPI == JH_EPI_GEGLU_BF16) {
#pragma unroll
            for (int i = 0; i < FB; i += 2) {
                const int slab = fw0 + i * 32;  // 64-aligned: [slab, slab+32) pairs with [slab+32, slab+64)
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
                const int slab = fw0 + i * 32;
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
    // Grouped order inside an XCD's band: GROUP token blocks are swept for
    // each feature block, so the ~64 tiles resident on one XCD share about
    // GROUP token blocks and 64/GROUP feature blocks of operands in its L2.
    constexpr int GROUP = 8;
    const int grp = tile / (GROUP * nF), gi = tile - grp * GROUP * nF;
    const int gh = min(GROUP, nTk - grp * GROUP);
    const int f0 = (gi / gh) * BF, t0 = (grp * GROUP + gi % gh) * BT;

    // Per-thread source rows for the global->LDS copies (fixed across K steps).
    // Rows past the end are clamped onto the last valid row: their products
    // land in accumulator rows the epilogue never stores, and the loads stay
    // unconditional, which keeps the compiler's vmcnt tracking exact (a
    // branch around a load makes it wait for every load in flight).
    const bf16_t* wsrc[CW];
    const bf16_t* xsrc[CX];
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        int c = tid + NT * i, row = c >> 3, kc = c & 7;
        int f = min(f0 + row, a.n - 1);
        wsrc[i] = a.w + (long)f * a.k + kc * 8;
    }
#pragma unroll
    for (int i = 0; i < CX; ++i) {
        int c = tid + NT * i, row = c >> 3, kc = c & 7;
        int t = min(t0 + row, a.rows - 1);
        long src = a.gather ? (long)a.gather[t] : (long)t;
        xsrc[i] = a.x + src * a.ldx + kc * 8;
    }

    struct Stage {
        u32x4 w[CW], x[CX];
    };
    auto gload = [&](Stage& s, int kt) {
        const int kb = kt * BK;
#pragma unroll
        for (int i = 0; i < CW; ++i) s.w[i] = *(const u32x4*)(wsrc[i] + kb);
#pragma unroll
        for (int i = 0; i < CX; ++i) s.x[i] = *(const u32x4*)(xsrc[i] + kb);
    };
    auto sstore = [&](const Stage& s, int buf) {
#pragma unroll
        for (int i = 0; i < CW; ++i) {
            int c = tid + NT * i;
            *(u32x4*)&sW[buf][c >> 3][(c & 7) * 8] = s.w[i];
        }
#pragma unroll
        for (int i = 0; i < CX; ++i) {
            int c = tid + NT * i;
            *(u32x4*)&sX[buf][c >> 3][(c & 7) * 8] = s.x[i];
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

    auto compute = [&](int buf) {
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
    };

    // K steps kt = 0..KT-1.  Tile kt is loaded into register stage kt%2 two
    // steps ahead and stored to LDS buffer kt%2 at the end of step kt-1.  The
    // prefetch index is clamped instead of skipped near the end (re-reading the
    // last tile from L2) so the steady-state loop carries no branches.
    const int KT = a.k / BK;
    Stage r0, r1;
    gload(r0, 0);
    gload(r1, min(1, KT - 1));
    sstore(r0, 0);
    __syncthreads();
    gload(r0, min(2, KT - 1));
    // One step: compute from LDS buf; stage `nxt` holds tile kt+1 -> LDS buf^1;
    // then refill `nxt` with tile kt+3.
    auto step = [&](int kt, Stage& nxt) {
        const int buf = kt & 1;
        compute(buf);
        sstore(nxt, buf ^ 1);
        gload(nxt, min(kt + 3, KT - 1));
        __syncthreads();
    };
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        step(kt, r1);
        step(kt + 1, r0);
    }
    if (kt < KT) compute(kt & 1);

    epilogue<EPI, FB, TB>(a, acc, f0 + wf * FPW, t0 + wt * TPW, lane);
}

// Tile shape: 128 features x 128 tokens, four waves of 64x64, two resident
// workgroups per CU (73.7 KB of LDS each).  Measured on MI355X against
// 256x256 (8 waves of 128x64, one workgroup per CU) and 256x128 (4 waves of
// 128x64): the two independent workgroups per CU hide each other's barrier
// and LDS latency, which outweighs the 25-50% fewer LDS bytes per MFMA of the
// wider wave tiles at one workgroup per CU.
template <int EPI>
void launch_cfg(const GemmArgs& a, hipStream_t s) {
    constexpr int BF = 128, BT = 128;
    const int blocks = ((a.n + BF - 1) / BF) * ((a.rows + BT - 1) / BT);
    JH_LAUNCH((gemm_kernel<EPI, BF, BT, 2, 2>), dim3(blocks), dim3(256), 0, s, a);
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
