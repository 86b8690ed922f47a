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
// Pipeline: workgroup tile 128 features x 128 tokens x BK=64, four waves of
// 64x64.  Operands go global -> LDS by buffer DMA (no register staging),
// double-buffered: the DMA of K step kt+1 runs under the MFMAs of step kt,
// one barrier per step, two resident workgroups per CU (64 KB LDS each); the
// epilogue stages the tile through the same LDS for row-contiguous stores.
// Outputs with more tiles than fit at once run persistent workgroups, which
// also prefetch each next tile under the current one.
//
// Tiles are dealt XCD-contiguously: MI355X hands workgroups round-robin to its
// 8 XCDs, so tile t goes to the workgroup whose id mod 8 selects the XCD that
// owns t's band; inside a band, tiles are grouped 8 token blocks at a time so
// the operands resident on one XCD fit its 4 MB L2.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <utility>

#include "../../include/julia1_hip_ops.h"
#include "kernels.hpp"
#include "rowvec.hpp"

namespace {

constexpr int BK = 64;

// Internal epilogue of the split-K partial pass: raw FP32 accumulators to the
// workspace (no bias), reduced and finished by splitk_reduce.
constexpr int EPI_PARTIAL = 100;
constexpr int SPLITK_MAX = 16;  // most K chunks of one split-K GEMM

// LDS chunk swizzle of operand row r (see gemm_kernel).
__device__ constexpr int swz(int r) { return (r >> 1) & 7; }

// Staging-row swizzle for rows of CPR 16-byte chunks: the 16 rows that a
// quarter-wave writes (one chunk each) land on 16 distinct 16-byte bank slots.
template <int CPR>
__device__ constexpr int oswz(int r) {
    return CPR == 16 ? (r & 15) : ((r >> 1) & 7);
}

// Epilogue of one wave's 64 x (32·TB) tile (features fw0.., tokens tw0..).
// acc[i][j][e] holds feature fw0 + i*32 + (e/4)*8 + g4 + e%4 of token
// tw0 + j*32 + lr.  Phase 1 applies the elementwise part in registers and
// writes the results to the wave's staging rows in LDS ([token][column]):
// FP32 for the FP32 outputs, already rounded to bf16 for the bf16 outputs
// (the same rounding of the same values, at half the LDS traffic); phase 2
// reads them back along rows so each store instruction writes whole
// 64/128/256-byte row segments instead of 32 scattered pieces.
template <int EPI, int TB = 2>
__device__ inline void epilogue(const GemmArgs& a, f32x16 (&acc)[2][TB], int fw0, int tw0, int lane, float* stage,
                                const f32x4* rope_c = nullptr, const f32x4* rope_s = nullptr) {
    constexpr int ROWS = TB * 32;  // staged token rows
    constexpr bool GEGLU = EPI == JH_EPI_GEGLU_BF16;
    constexpr bool F32OUT = EPI == JH_EPI_RESID_F32 || EPI == JH_EPI_BIAS_F32 || EPI == EPI_PARTIAL;
    constexpr bool BIASED = EPI == JH_EPI_BIAS_BF16 || EPI == JH_EPI_BIAS_RELU_BF16 || EPI == JH_EPI_BIAS_F32;
    constexpr int OW = GEGLU ? 32 : 64;  // output columns of the wave tile
    constexpr int CPR = OW / 4;          // 16-byte FP32 chunks per staging row
    const int g4 = (lane >> 5) * 4, lr = lane & 31;
    auto put = [&](int row, int chunk, f32x4 v) { *(f32x4*)&stage[row * OW + ((chunk ^ oswz<CPR>(row)) * 4)] = v; };
    // bf16 staging rows: OW/8 16-byte chunks, XOR-swizzled by the row so that
    // the 8-byte writes of 64 lanes (32 rows x 2 halves of one chunk) and the
    // 16-byte row reads of each quarter-wave both spread over all banks.
    constexpr int BCPR = OW / 8;
    bf16_t* const bstage = (bf16_t*)stage;
    auto bswz = [](int r) { return BCPR == 8 ? (r >> 1) & 7 : (r >> 2) & 3; };
    auto putb = [&](int row, int fl, f32x4 v) {  // columns fl .. fl+3, fl % 4 == 0
        *(u32x2*)&bstage[row * OW + (((fl >> 3) ^ bswz(row)) * 8) + (fl & 4)] =
            u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    };
    const long col0 = a.col + (GEGLU ? fw0 / 2 : fw0);

    // Residual: all 16 of this lane's old FP32 chunks are loaded before the
    // staging pass (rows past the end re-read the last row and are not
    // stored), so their latency overlaps it instead of serialising the
    // read-modify-write loop one row pass at a time.
    constexpr int RPASS = ROWS / 4;  // 4-row passes over the staged rows
    f32x4 old[EPI == JH_EPI_RESID_F32 ? RPASS : 1];
    if constexpr (EPI == JH_EPI_RESID_F32) {
#pragma unroll
        for (int p = 0; p < RPASS; ++p) {
            const int t = min(tw0 + (lane >> 4) + 4 * p, a.rows - 1);
            old[p] = *(const f32x4*)((const float*)a.out + (long)t * a.ldo + col0 + (lane & 15) * 4);
        }
    }

#pragma unroll
    for (int j = 0; j < TB; ++j) {
        const int tl = j * 32 + lr;
        if constexpr (EPI == JH_EPI_ROPE_BF16) {
            const bool rot = fw0 < a.rope_cols;
            const long p = rot && !rope_c ? (long)(a.pos[min(tw0 + tl, a.rows - 1)] & 0xffff) * 32 : 0;
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int d = qd * 8 + g4;
                f32x4 lo, hi;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lo[e] = acc[0][j][qd * 4 + e];
                    hi[e] = acc[1][j][qd * 4 + e];
                }
                if (rot) {
                    const f32x4 c = rope_c ? rope_c[j * 4 + qd] : *(const f32x4*)(a.cos_t + p + d);
                    const f32x4 s = rope_s ? rope_s[j * 4 + qd] : *(const f32x4*)(a.sin_t + p + d);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float l = lo[e], h = hi[e];
                        rope_rotate(l, h, c[e], s[e]);
                        lo[e] = l;
                        hi[e] = h;
                    }
                }
                putb(tl, d, lo);
                putb(tl, 32 + d, hi);
            }
        } else if constexpr (GEGLU) {
            // Rows [fw0, fw0+32) are gate, [fw0+32, fw0+64) up, for outputs fw0/2 + [0, 32).
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                const int d = qd * 8 + g4;
                f32x4 g;
#pragma unroll
                for (int e = 0; e < 4; ++e) g[e] = gelu_erf(acc[0][j][qd * 4 + e]) * acc[1][j][qd * 4 + e];
                putb(tl, d, g);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const int fl = i * 32 + qd * 8 + g4;
                    f32x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = acc[i][j][qd * 4 + e];
                    if (BIASED || (EPI == JH_EPI_RESID_F32 && a.bias)) {
                        const f32x4 bb = *(const f32x4*)(a.bias + fw0 + fl);
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            v[e] += bb[e];
                            if constexpr (EPI == JH_EPI_BIAS_RELU_BF16) v[e] = fmaxf(v[e], 0.0f);
                        }
                    }
                    if constexpr (F32OUT) put(tl, fl / 4, v);
                    else putb(tl, fl, v);
                }
        }
    }

    if constexpr (F32OUT) {
        // 16 lanes per 256-byte row, 4 rows per pass.
        const int q = lane & 15;
#pragma unroll
        for (int p = 0; p < RPASS; ++p) {
            const int rr = (lane >> 4) + 4 * p, t = tw0 + rr;
            if (t < a.rows) {
                const f32x4 v = *(const f32x4*)&stage[rr * OW + ((q ^ oswz<CPR>(rr)) * 4)];
                float* o = (float*)a.out + (long)t * a.ldo + col0 + q * 4;
                if constexpr (EPI == JH_EPI_RESID_F32) {
                    f32x4 r = old[p];
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[e] += v[e];
                    *(f32x4*)o = r;
                } else {
                    *(f32x4*)o = v;
                }
            }
        }
    } else {
        // OW/8 lanes per bf16 output row (16 bytes each), 64/(OW/8) rows per pass.
        constexpr int LPR = BCPR, RPP = 64 / LPR;
        const int q = lane % LPR;
#pragma unroll 4
        for (int rr = lane / LPR; rr < ROWS; rr += RPP) {
            const int t = tw0 + rr;
            if (t >= a.rows) break;
            *(u32x4*)((bf16_t*)a.out + (long)t * a.ldo + col0 + q * 8) =
                *(const u32x4*)&bstage[rr * OW + ((q ^ bswz(rr)) * 8)];
        }
    }
}

// Operands reach LDS by DMA: buffer_load_dwordx4 ... lds (global_load_lds_dwordx4
// with 64-bit per-lane addresses for row-gathered X) writes 64 lanes x 16 B to
// one contiguous 1 KB LDS block at M0 (lane i at +16i, verified on gfx950).
// The buffer form (per-lane 32-bit offsets from a per-tile base, scalar K
// offset) measured ~8% faster than the 64-bit global form in this kernel.
// LDS rows cannot be padded, so lane i loads the global chunk that belongs in
// its slot under an XOR swizzle (physical chunk = logical chunk ^ ((row >> 1)
// & 7) for 128-byte rows).  Measured on gfx950, a 16-byte-per-lane LDS read
// runs at full rate only when each quarter-wave (16 lanes) touches 256
// distinct bytes of the 64 x 4-byte banks: with this swizzle the 16 rows a
// quarter-wave reads fall into 16 distinct (row parity, chunk) slots (the
// plain row & 7 swizzle puts rows r and r+8 on the same banks and halves LDS
// read bandwidth).  The DMA is issued with inline asm so the compiler does not
// insert its conservative vmcnt(0) before every LDS read; the wait for a stage
// is explicit.
template <int EPI, bool GATHER>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_kernel(GemmArgs a) {
    constexpr int BF = 128, BT = 128, FB = 2, TB = 2, NS = 2;
    constexpr int CPR = BK / 8;           // 16-byte chunks per row (8)
    constexpr int RPI = 64 / CPR;         // rows per 1 KB DMA instruction (8)
    constexpr int IPW = BF / RPI / 4;     // DMA instructions per wave per operand per stage (4)
    constexpr int STAGE = BF * BK;        // bf16 elements per operand per stage
    // Operand stages during the K loop; the four waves' 16 KB epilogue staging
    // rows afterwards.
    __shared__ __align__(1024) bf16_t smem[2 * NS * STAGE];
    bf16_t* const sW = smem;
    bf16_t* const sX = smem + NS * STAGE;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nF = (a.n + BF - 1) / BF, nTk = (a.rows + BT - 1) / BT, ntiles = nF * nTk;
    // Split-K partial pass: workgroup blockIdx.x covers tile blockIdx.x % ntiles
    // and K steps [split·kt_chunk, (split+1)·kt_chunk).
    const int split = EPI == EPI_PARTIAL ? (int)blockIdx.x / ntiles : 0;
    const int b = EPI == EPI_PARTIAL ? (int)blockIdx.x - split * ntiles : (int)blockIdx.x;
    const int xcd = b & 7, local = b >> 3, q8 = ntiles >> 3, r8 = ntiles & 7;
    const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    // Grouped order inside an XCD's band: GROUP token blocks are swept for
    // each feature block, so the ~64 tiles resident on one XCD share about
    // GROUP token blocks and 64/GROUP feature blocks of operands in its L2.
    constexpr int GROUP = 8;
    const int grp = tile / (GROUP * nF), gi = tile - grp * GROUP * nF;
    const int gh = min(GROUP, nTk - grp * GROUP);
    const int f0 = (gi / gh) * BF, t0 = (grp * GROUP + gi % gh) * BT;

    // Per-lane DMA sources: rows past the end are clamped onto the last valid
    // row (their products land in accumulator rows the epilogue never stores).
    // W (and X unless row-gathered) load through buffer resources based at the
    // tile (32-bit per-lane offsets plus a scalar K offset); gathered X rows
    // use 64-bit per-lane addresses.
    const bf16_t* wt0 = a.w + (long)f0 * a.k;
    const bf16_t* xt0 = a.x + (long)t0 * a.ldx;
    const i32x4 rw = make_rsrc(wt0, (uint64_t)(a.n - f0) * a.k * 2);
    const i32x4 rx = make_rsrc(xt0, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)a.k * 2);
    uint32_t woff[IPW], xoff[IPW];
    const bf16_t* xsrc[GATHER ? IPW : 1];
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
        const int lrow = (wave * IPW + j) * RPI + lane / CPR;
        const int c = (lane % CPR) ^ swz(lrow);
        woff[j] = (uint32_t)((min(f0 + lrow, a.n - 1) - f0) * a.k + c * 8) * 2;
        const int t = min(t0 + lrow, a.rows - 1);
        if constexpr (GATHER) xsrc[j] = a.x + (long)a.gather[t] * a.ldx + c * 8;
        else xoff[j] = (uint32_t)((t - t0) * (long)a.ldx + c * 8) * 2;
    }
    // LDS byte offsets (low 32 bits of the generic LDS address) of this wave's blocks.
    const uint32_t wl0 = (uint32_t)(uintptr_t)&sW[wave * IPW * 512];
    const uint32_t xl0 = (uint32_t)(uintptr_t)&sX[wave * IPW * 512];
    auto issue = [&](int kt, int st) {
        const uint32_t kb = (uint32_t)kt * BK * 2;  // bytes
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const uint32_t lw = __builtin_amdgcn_readfirstlane(wl0 + (st * STAGE + j * 512) * 2);
            const uint32_t lx = __builtin_amdgcn_readfirstlane(xl0 + (st * STAGE + j * 512) * 2);
            asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lw), "v"(woff[j]), "s"(rw), "s"(kb)
                         : "memory");
            if constexpr (GATHER)
                asm volatile("global_load_lds_dwordx4 %1, off" ::"{m0}"(lx), "v"(xsrc[j] + kb / 2) : "memory");
            else
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lx), "v"(xoff[j]), "s"(rx), "s"(kb)
                             : "memory");
        }
    };

    const int wf = wave & 1, wt = wave >> 1, lr = lane & 31, lg = lane >> 5;
    f32x16 acc[FB][TB];
#pragma unroll
    for (int i = 0; i < FB; ++i)
#pragma unroll
        for (int j = 0; j < TB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // Step kt: wait for this wave's DMA of stage kt%2, barrier (all waves' data
    // landed, and everyone finished reading the other stage), then start the
    // DMA of step kt+1 into the other stage and run the MFMAs of step kt.
    const int kt0 = EPI == EPI_PARTIAL ? split * a.kt_chunk : 0;
    const int KT = EPI == EPI_PARTIAL ? min(a.k / BK, kt0 + a.kt_chunk) : a.k / BK;
    issue(kt0, 0);
    for (int kt = kt0; kt < KT; ++kt) {
        const int st = (kt - kt0) & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (kt + 1 < KT) issue(kt + 1, st ^ 1);
        const bf16_t* W = sW + st * STAGE;
        const bf16_t* X = sX + st * STAGE;
        // Fragments are double-buffered in registers: the LDS reads of slice
        // ks+1 are in flight while the MFMAs of slice ks run.
        bf16x8 af[2][FB], bx[2][TB];
        auto load = [&](int ks, int s) {
            const int c = ks * 2 + lg;
#pragma unroll
            for (int i = 0; i < FB; ++i) {
                const int r = wf * 64 + i * 32 + lr;
                af[s][i] = *(const bf16x8*)&W[r * BK + ((c ^ swz(r)) * 8)];
            }
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                const int r = wt * 64 + j * 32 + lr;
                bx[s][j] = *(const bf16x8*)&X[r * BK + ((c ^ swz(r)) * 8)];
            }
        };
        // Order pinned with scheduling fences: reads of slices 0 and 1, then
        // per slice its MFMAs followed by the reads of the slice two ahead
        // into the registers those MFMAs just consumed (left to itself the
        // compiler reuses one fragment set and waits out every read).
        load(0, 0);
        load(1, 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int s = ks & 1;
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FB; ++i)
#pragma unroll
                for (int j = 0; j < TB; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][i], bx[s][j], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (ks + 2 < BK / 16) load(ks + 2, s);
        }
    }
    __syncthreads();  // every wave is done reading the operand stages
    if (f0 + wf * 64 >= a.n) return;
    if constexpr (EPI == EPI_PARTIAL) {
        GemmArgs e = a;
        e.out = a.partial + (size_t)split * a.rows * a.n;
        e.ldo = a.n;
        e.col = 0;
        epilogue<EPI>(e, acc, f0 + wf * 64, t0 + wt * 64, lane, (float*)smem + wave * 4096);
    } else {
        epilogue<EPI>(a, acc, f0 + wf * 64, t0 + wt * 64, lane, (float*)smem + wave * 4096);
    }
}

// Persistent variant of gemm_kernel for outputs with more tiles than resident
// workgroups (two per CU): gridDim.x workgroups walk the tiles g, g + G, ...
// (G a multiple of 8, so a workgroup stays in its XCD's band).  The DMA of the
// next tile's first K step is issued at the current tile's last step into the
// buffer that step does not read, so it lands under that step's MFMAs instead
// of in front of the next tile.  Each wave waits for it before its epilogue,
// whose stores (counted by vmcnt too) are then never waited on; the epilogue
// stages through the last step's buffers, 8 KB per wave, in two 32-row passes.
// Same products in the same K order as gemm_kernel, so results are identical.
// BT = 128 or 192 tokens per tile (waves of 64 features x BT/2 tokens): the
// 128x192 tile moves 17% fewer operand bytes per MFMA in 80 KB of LDS, which
// still leaves two workgroups per CU.
template <int EPI, int BT = 128>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void gemm_persist_kernel(GemmArgs a) {
    constexpr int BF = 128, FB = 2, TB = BT / 64;
    constexpr int CPR = BK / 8, RPI = 64 / CPR;
    constexpr int IPW = BF / RPI / 4, XPW = BT / RPI / 4;  // W / X DMA instructions per wave and stage
    constexpr int STAGE = BF * BK, XSTAGE = BT * BK;
    __shared__ __align__(1024) bf16_t smem[2 * STAGE + 2 * XSTAGE];
    bf16_t* const sW = smem;
    bf16_t* const sX = smem + 2 * STAGE;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nF = (a.n + BF - 1) / BF, nTk = (a.rows + BT - 1) / BT, ntiles = nF * nTk;
    auto coords = [&](int b, int& f0, int& t0) {
        const int xcd = b & 7, local = b >> 3, q8 = ntiles >> 3, r8 = ntiles & 7;
        const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
        constexpr int GROUP = 8;
        const int grp = tile / (GROUP * nF), gi = tile - grp * GROUP * nF;
        const int gh = min(GROUP, nTk - grp * GROUP);
        f0 = (gi / gh) * BF;
        t0 = (grp * GROUP + gi % gh) * BT;
    };
    struct Src {
        i32x4 rw, rx;
        uint32_t woff[IPW], xoff[XPW];
    };
    auto setup = [&](int f0, int t0, Src& s) {
        s.rw = make_rsrc(a.w + (long)f0 * a.k, (uint64_t)(a.n - f0) * a.k * 2);
        s.rx = make_rsrc(a.x + (long)t0 * a.ldx, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)a.k * 2);
#pragma unroll
        for (int j = 0; j < IPW; ++j) {
            const int lrow = (wave * IPW + j) * RPI + lane / CPR;
            const int c = (lane % CPR) ^ swz(lrow);
            s.woff[j] = (uint32_t)((min(f0 + lrow, a.n - 1) - f0) * a.k + c * 8) * 2;
        }
#pragma unroll
        for (int j = 0; j < XPW; ++j) {
            const int lrow = (wave * XPW + j) * RPI + lane / CPR;
            const int c = (lane % CPR) ^ swz(lrow);
            const int t = min(t0 + lrow, a.rows - 1);
            s.xoff[j] = (uint32_t)((t - t0) * (long)a.ldx + c * 8) * 2;
        }
    };
    const uint32_t wl0 = (uint32_t)(uintptr_t)&sW[wave * IPW * 512];
    const uint32_t xl0 = (uint32_t)(uintptr_t)&sX[wave * XPW * 512];
    auto issue = [&](const Src& s, int kt, int st) {
        const uint32_t kb = (uint32_t)kt * BK * 2;
#pragma unroll
        for (int j = 0; j < (IPW > XPW ? IPW : XPW); ++j) {
            if (j < IPW) {
                const uint32_t lw = __builtin_amdgcn_readfirstlane(wl0 + (st * STAGE + j * 512) * 2);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lw), "v"(s.woff[j]), "s"(s.rw),
                             "s"(kb)
                             : "memory");
            }
            if (j < XPW) {
                const uint32_t lx = __builtin_amdgcn_readfirstlane(xl0 + (st * XSTAGE + j * 512) * 2);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lx), "v"(s.xoff[j]), "s"(s.rx),
                             "s"(kb)
                             : "memory");
            }
        }
    };
    const int wf = wave & 1, wt = wave >> 1, lr = lane & 31, lg = lane >> 5;
    const int G = gridDim.x, KT = a.k / BK;
    int cur = blockIdx.x, f0, t0, base = 0;
    // A grid larger than the tile count (launch_cfg never makes one) would
    // otherwise compute tile coordinates past the matrix for the extra
    // workgroups and aim their DMA outside the operands.
    if (cur >= ntiles) return;
    coords(cur, f0, t0);
    Src sc;
    setup(f0, t0, sc);
    issue(sc, 0, 0);
    bool first = true;
    while (true) {
        const int nxt = cur + G;
        const bool has_next = nxt < ntiles;
        int nf0 = 0, nt0 = 0;
        Src sn = sc;
        if (has_next) {
            coords(nxt, nf0, nt0);
            setup(nf0, nt0, sn);
        }
        // RoPE epilogue: this lane's cos/sin values for its two tokens are
        // loaded before the K loop, so their latency (position, then table)
        // runs under the MFMAs instead of in front of the epilogue.
        // (two tokens only: with three the registers do not fit two waves per SIMD)
        constexpr bool PRE = EPI == JH_EPI_ROPE_BF16 && TB == 2;
        f32x4 rc[PRE ? TB * 4 : 1], rs[PRE ? TB * 4 : 1];
        if constexpr (PRE) {
            if (f0 + wf * 64 < a.rope_cols) {
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    const long p = (long)(a.pos[min(t0 + wt * (BT / 2) + j * 32 + lr, a.rows - 1)] & 0xffff) * 32;
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        rc[j * 4 + qd] = *(const f32x4*)(a.cos_t + p + qd * 8 + lg * 4);
                        rs[j * 4 + qd] = *(const f32x4*)(a.sin_t + p + qd * 8 + lg * 4);
                    }
                }
            }
        }
        f32x16 acc[FB][TB];
#pragma unroll
        for (int i = 0; i < FB; ++i)
#pragma unroll
            for (int j = 0; j < TB; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int kt = 0; kt < KT; ++kt) {
            const int st = (base + kt) & 1;
            // a later tile's step-0 DMA was waited for before the previous epilogue
            if (kt > 0 || first) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (kt + 1 < KT) issue(sc, kt + 1, st ^ 1);
            else if (has_next) issue(sn, 0, st ^ 1);
            const bf16_t* W = sW + st * STAGE;
            const bf16_t* X = sX + st * XSTAGE;
            bf16x8 af[2][FB], bx[2][TB];
            auto load = [&](int ks, int s) {
                const int c = ks * 2 + lg;
#pragma unroll
                for (int i = 0; i < FB; ++i) {
                    const int r = wf * 64 + i * 32 + lr;
                    af[s][i] = *(const bf16x8*)&W[r * BK + ((c ^ swz(r)) * 8)];
                }
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    const int r = wt * (BT / 2) + j * 32 + lr;
                    bx[s][j] = *(const bf16x8*)&X[r * BK + ((c ^ swz(r)) * 8)];
                }
            };
            load(0, 0);
            load(1, 1);
#pragma unroll
            for (int ks = 0; ks < BK / 16; ++ks) {
                const int s = ks & 1;
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < FB; ++i)
#pragma unroll
                    for (int j = 0; j < TB; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][i], bx[s][j], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (ks + 2 < BK / 16) load(ks + 2, s);
            }
        }
        const int st_last = (base + KT - 1) & 1;
        __syncthreads();  // every wave is done reading the last step's buffers
        if (has_next) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        float* stg = wave < 2 ? (float*)(sW + st_last * STAGE) + wave * 2048
                              : (float*)(sX + st_last * XSTAGE) + (wave - 2) * 2048;
        if (f0 + wf * 64 < a.n) {
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                f32x16 part[2][1] = {{acc[0][j]}, {acc[1][j]}};
                const int tw = t0 + wt * (BT / 2) + j * 32;
                if constexpr (PRE)
                    epilogue<EPI, 1>(a, part, f0 + wf * 64, tw, lane, stg, rc + j * 4, rs + j * 4);
                else
                    epilogue<EPI, 1>(a, part, f0 + wf * 64, tw, lane, stg);
            }
        }
        if (!has_next) break;
        cur = nxt;
        f0 = nf0;
        t0 = nt0;
        sc = sn;
        base = (base + KT) & 1;
        first = false;
    }
}

// Eight-wave variant for wide outputs (N >= 1024): one workgroup per CU owns
// a 256-feature x BT-token tile (BT = 192 or 256), eight waves of 64
// features x BT/2 tokens (on a tile 32 tokens shorter, waves 0-3 take 32
// tokens fewer).  The operand DMA of a K step is 1 KB per
// instruction through the texture addresser (TA), which drains one
// instruction per ~16 cycles per CU; a wave blocks while its instructions
// wait there.  When all waves issue their share right after the step's
// barrier, every wave stalls for most of the burst before its first MFMA
// (measured ~600-700 cycles per step).  Here waves 0-3 (one per SIMD) issue
// all of a step's DMA, and waves 4-7, which share those SIMDs, start their
// MFMAs at once; waves 0-3 compute after their burst, while 4-7 wait at the
// next barrier.  The tile moves half the operand bytes per MFMA of a
// 128x128 tile.  Each wave stages its epilogue through 8 KB (FP32 outputs)
// or 4 KB (bf16 outputs) of the last step's buffers, plus a slack block when
// those are too small.  Same products in the same K order as gemm_kernel:
// results are identical.
//
// RoPE with 192-token tiles: the tile's cos/sin table rows (192 tokens x 32
// f32 each, 48 KB) are gathered into LDS by the loader waves' DMA during the
// second-to-last K step, and every wave's epilogue reads them from there.
// Loaded from global memory by each wave instead, the four feature waves of a
// token block would each fetch the same rows: 192 KB per tile through the
// texture addresser, twice the tile's output bytes, with the epilogue waiting
// on them (measured: 5.3-5.9 us per tile against 2.2-2.9 us for a plain store).
template <int EPI, int BT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_big_kernel(GemmArgs a) {
    constexpr int BF = 256, FB = 2, TB = BT / 64;
    constexpr int NW = BF / 32, NX = BT / 32;          // DMA instructions per loader wave and stage (W, X)
    constexpr int WSTAGE = BF * BK, XSTAGE = BT * BK;  // bf16 elements per stage
    constexpr bool F32OUT = EPI == JH_EPI_RESID_F32 || EPI == JH_EPI_BIAS_F32;
    constexpr int STG = F32OUT ? 4096 : 2048;           // bf16 elements of staging per wave
    constexpr int SLACK = 8 * STG > WSTAGE + XSTAGE ? 8 * STG - (WSTAGE + XSTAGE) : 0;
    constexpr bool RLDS = EPI == JH_EPI_ROPE_BF16 && BT == 192;  // cos/sin rows staged in LDS
    constexpr int CSROWS = RLDS ? BT : 0;                        // 128-byte table rows per table
    constexpr int NCS = CSROWS / 8 / 4;                          // DMA instructions per loader wave per table
    __shared__ __align__(1024) bf16_t smem[2 * WSTAGE + 2 * XSTAGE + SLACK + 2 * CSROWS * 64];
    bf16_t* const sW = smem;
    bf16_t* const sX = smem + 2 * WSTAGE;
    bf16_t* const sSlack = smem + 2 * WSTAGE + 2 * XSTAGE;
    float* const sCos = (float*)(sSlack + SLACK);  // [CSROWS][32], 16-byte chunks swizzled by swz(row)
    float* const sSin = sCos + CSROWS * 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool loader = wave < 4;
    // Token tiles come in two phases: rows [0, mix) in BT-token tiles, then
    // (mix > 0) the rest in (BT-32)-token tiles, so that the last round of
    // resident workgroups carries smaller tiles instead of leaving CUs idle.
    // Each phase is dealt as its own round-robin over the grid.
    const int nF = (a.n + BF - 1) / BF;
    const int mix = a.mix_rows;
    const int nT[2] = {((mix > 0 ? mix : a.rows) + BT - 1) / BT, mix > 0 ? (a.rows - mix + BT - 33) / (BT - 32) : 0};
    const int nTiles[2] = {nF * nT[0], nF * nT[1]};
    // Tile b of phase ph: f0, t0 and its token height ht.
    auto coords = [&](int ph, int b, int& f0, int& t0, int& ht) {
        const int ntiles = nTiles[ph], nTk = nT[ph];
        ht = ph ? BT - 32 : BT;
        const int xcd = b & 7, local = b >> 3, q8 = ntiles >> 3, r8 = ntiles & 7;
        const int tile = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
        constexpr int GROUP = 4;
        const int grp = tile / (GROUP * nF), gi = tile - grp * GROUP * nF;
        const int gh = min(GROUP, nTk - grp * GROUP);
        f0 = (gi / gh) * BF;
        t0 = (ph ? mix : 0) + (grp * GROUP + gi % gh) * ht;
    };
    // Loader wave w's instruction j fills operand rows 32j + 8w .. +7 (lane i:
    // row 32j + 8w + i/8, swizzled chunk); rows past the end of W or X fall
    // outside the buffer resource's range, read as zeros, and land in
    // accumulator rows that are never stored.
    const int lrow = (wave & 3) * 8 + lane / 8;  // row within each 32-row block
    const uint32_t lchunk = (uint32_t)(((lane & 7) ^ swz(lrow)) * 16);
    struct Src {
        i32x4 rw, rx;
    };
    auto setup = [&](int f0, int t0, Src& s) {
        s.rw = make_rsrc(a.w + (long)f0 * a.k, (uint64_t)(a.n - f0) * a.k * 2);
        s.rx = make_rsrc(a.x + (long)t0 * a.ldx, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)a.k * 2);
    };
    const uint32_t woff = (uint32_t)lrow * a.k * 2 + lchunk, xoff = (uint32_t)(lrow * a.ldx) * 2 + lchunk;
    const uint32_t wstep = 32u * a.k * 2, xstep = 32u * (uint32_t)a.ldx * 2;  // bytes per 32 rows
    const uint32_t wl0 = (uint32_t)(uintptr_t)&sW[(wave & 3) * 8 * 64];
    const uint32_t xl0 = (uint32_t)(uintptr_t)&sX[(wave & 3) * 8 * 64];
    // X rows [ht, BT) of a short tile are not loaded.
    auto issue = [&](const Src& s, int kt, int st, int ht) {
        const uint32_t kb = (uint32_t)kt * BK * 2;
#pragma unroll
        for (int j = 0; j < (NW > NX ? NW : NX); ++j) {
            if (j < NW) {
                const uint32_t lw = __builtin_amdgcn_readfirstlane(wl0 + (st * WSTAGE + j * 32 * 64) * 2);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lw), "v"(woff + j * wstep),
                             "s"(s.rw), "s"(kb)
                             : "memory");
            }
            if (j < NX && (j < NX - 1 || ht == BT)) {
                const uint32_t lx = __builtin_amdgcn_readfirstlane(xl0 + (st * XSTAGE + j * 32 * 64) * 2);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lx), "v"(xoff + j * xstep),
                             "s"(s.rx), "s"(kb)
                             : "memory");
            }
        }
    };
    const int wf = wave & 3, lr = lane & 31, lg = lane >> 5;
    const int G = gridDim.x, KT = a.k / BK;
    // Waves 0-3 multiply the tile's first 32·TB tokens (32·(TB-1) on a short
    // tile), waves 4-7 the next 32·TB.
    int ph = 0, cur = blockIdx.x, f0, t0, ht, base = 0;
    if (cur >= nTiles[0]) {
        ph = 1;
        if (cur >= nTiles[1]) return;
    }
    coords(ph, cur, f0, t0, ht);
    Src sc;
    setup(f0, t0, sc);
    if (loader) issue(sc, 0, 0, ht);
    bool first = true;
    while (true) {
        int nph = ph, nxt = cur + G;
        if (nxt >= nTiles[ph] && ph == 0) nph = 1, nxt = blockIdx.x;
        const bool has_next = nxt < nTiles[nph];
        int nf0 = 0, nt0 = 0, nht = BT;
        Src sn = sc;
        if (has_next) {
            coords(nph, nxt, nf0, nt0, nht);
            setup(nf0, nt0, sn);
        }
        const int lb = ht == BT ? TB : TB - 1;           // 32-token blocks of the loader waves
        const int toff = loader ? 0 : lb * 32;          // this wave's first token in the tile
        const bool full = !loader || ht == BT;          // this wave multiplies all TB blocks
        // RoPE with 192-token tiles (RLDS): the loader waves gather the tile's
        // cos/sin rows into LDS during the last K steps, so the epilogue, which
        // every wave of the CU runs at once, reads them from LDS instead of
        // starting on two dependent global loads.  (256-token tiles keep the
        // loads inside the epilogue: with the staging their registers do not
        // fit two waves per SIMD.)
        constexpr bool ROPE = RLDS;
        const bool rot = ROPE && f0 + wf * 64 < a.rope_cols;
        // RLDS: loader wave w gathers table rows [NCS*8*w, NCS*8*(w+1)) of the
        // tile's tokens, lane i row 8j + i/8 of its instruction j, the 16-byte
        // chunk that belongs in slot i%8 of that row under the swizzle.
        const bool rot_tile = RLDS && loader && f0 < a.rope_cols;
        uint32_t csoff[RLDS ? NCS : 1];
        if constexpr (RLDS) {
            if (rot_tile) {
#pragma unroll
                for (int j = 0; j < NCS; ++j) {
                    const int r = (wave * NCS + j) * 8 + (lane >> 3);
                    csoff[j] = (uint32_t)(a.pos[min(t0 + r, a.rows - 1)] & 0xffff) * 128 +
                               (uint32_t)(((lane & 7) ^ swz(r)) * 16);
                }
            }
        }
        auto rope_dma = [&]() {
            if constexpr (RLDS) {
                if (rot_tile) {
                    const i32x4 rcos = make_rsrc(a.cos_t, 65536ull * 128), rsin = make_rsrc(a.sin_t, 65536ull * 128);
#pragma unroll
                    for (int j = 0; j < NCS; ++j) {
                        const uint32_t lc = __builtin_amdgcn_readfirstlane(
                            (uint32_t)(uintptr_t)&sCos[(wave * NCS + j) * 8 * 32]);
                        const uint32_t ls = __builtin_amdgcn_readfirstlane(
                            (uint32_t)(uintptr_t)&sSin[(wave * NCS + j) * 8 * 32]);
                        asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(lc), "v"(csoff[j]),
                                     "s"(rcos), "s"(0)
                                     : "memory");
                        asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(ls), "v"(csoff[j]),
                                     "s"(rsin), "s"(0)
                                     : "memory");
                    }
                }
            }
        };
        f32x4 rc[4], rs[4];
        auto rope_load = [&](int j) {
            if constexpr (RLDS) {
                if (rot) {
                    const int r = toff + j * 32 + lr;
#pragma unroll
                    for (int qd = 0; qd < 4; ++qd) {
                        rc[qd] = *(const f32x4*)&sCos[r * 32 + ((qd * 2 + lg) ^ swz(r)) * 4];
                        rs[qd] = *(const f32x4*)&sSin[r * 32 + ((qd * 2 + lg) ^ swz(r)) * 4];
                    }
                }
            }
        };
        f32x16 acc[FB][TB];
#pragma unroll
        for (int i = 0; i < FB; ++i)
#pragma unroll
            for (int j = 0; j < TB; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
        for (int kt = 0; kt < KT; ++kt) {
            const int st = (base + kt) & 1;
            if (kt > 0 || first) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (loader) {
                if (kt + 1 < KT) issue(sc, kt + 1, st ^ 1, ht);
                else if (has_next) issue(sn, 0, st ^ 1, nht);
                // waited for at the next step's start (or before the epilogue when KT == 1)
                if (kt == (KT >= 2 ? KT - 2 : 0)) rope_dma();
            }
            const bf16_t* W = sW + st * WSTAGE;
            const bf16_t* X = sX + st * XSTAGE;
            bf16x8 af[2][FB], bx[2][TB];
            auto load = [&](int ks, int s) {
                const int c = ks * 2 + lg;
#pragma unroll
                for (int i = 0; i < FB; ++i) {
                    const int r = wf * 64 + i * 32 + lr;
                    af[s][i] = *(const bf16x8*)&W[r * BK + ((c ^ swz(r)) * 8)];
                }
#pragma unroll
                for (int j = 0; j < TB; ++j) {
                    const int r = toff + j * 32 + lr;
                    bx[s][j] = *(const bf16x8*)&X[r * BK + ((c ^ swz(r)) * 8)];
                }
            };
            load(0, 0);
            load(1, 1);
#pragma unroll
            for (int ks = 0; ks < BK / 16; ++ks) {
                const int s = ks & 1;
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < FB; ++i)
#pragma unroll
                    for (int j = 0; j < TB; ++j)
                        if (j < TB - 1 || full)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][i], bx[s][j], acc[i][j], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (ks + 2 < BK / 16) load(ks + 2, s);
            }
        }
        const int st_last = (base + KT - 1) & 1;
        // With one K step the cos/sin rows were issued in it: they land before the barrier.
        if (RLDS && KT == 1 && loader) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // every wave is done reading the last step's buffers
        if (has_next) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if constexpr (RLDS) rope_load(0);
        // Staging per wave: the last step's W buffer, then its X buffer, then
        // the slack block.
        const int so = wave * STG;
        bf16_t* const sbase = so < WSTAGE ? sW + st_last * WSTAGE + so
                              : so < WSTAGE + XSTAGE ? sX + st_last * XSTAGE + (so - WSTAGE)
                                                     : sSlack + (so - WSTAGE - XSTAGE);
        float* const stg = (float*)sbase;
        if (f0 + wf * 64 < a.n) {
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if (j == TB - 1 && !full) break;
                f32x16 part[2][1] = {{acc[0][j]}, {acc[1][j]}};
                if constexpr (ROPE) {
                    if (j > 0) rope_load(j);
                    epilogue<EPI, 1>(a, part, f0 + wf * 64, t0 + toff + j * 32, lane, stg, rc, rs);
                } else {
                    epilogue<EPI, 1>(a, part, f0 + wf * 64, t0 + toff + j * 32, lane, stg);
                }
            }
        }
        if (!has_next) break;
        ph = nph;
        cur = nxt;
        f0 = nf0;
        t0 = nt0;
        ht = nht;
        sc = sn;
        base = (base + KT) & 1;
        first = false;
    }
}

// Elementwise epilogue of FP32 sums for one output row t, features f .. f+3
// (epilogues without a 64-feature pairing).
template <int EPI>
__device__ inline void finish_one(const GemmArgs& a, long t, int f, f32x4 v) {
    const bool biased = EPI == JH_EPI_BIAS_BF16 || EPI == JH_EPI_BIAS_RELU_BF16 || EPI == JH_EPI_BIAS_F32 ||
                        (EPI == JH_EPI_RESID_F32 && a.bias);
    if (biased) {
        const f32x4 bb = *(const f32x4*)(a.bias + f);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] += bb[e];
            if constexpr (EPI == JH_EPI_BIAS_RELU_BF16) v[e] = fmaxf(v[e], 0.0f);
        }
    }
    const long c = a.col + f;
    if constexpr (EPI == JH_EPI_RESID_F32) {
        float* o = (float*)a.out + t * a.ldo + c;
        f32x4 r = *(const f32x4*)o;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] += v[e];
        *(f32x4*)o = r;
    } else if constexpr (EPI == JH_EPI_BIAS_F32) {
        *(f32x4*)((float*)a.out + t * a.ldo + c) = v;
    } else {
        *(u32x2*)((bf16_t*)a.out + t * a.ldo + c) = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    }
}

// The same for features slab + 4q .. +3 (lo) and slab + 32 + 4q .. +3 (hi) of
// a 64-feature block: the RoPE pair (d, d+32) and the GEGLU pair (gate, up)
// of an output are both here.
template <int EPI>
__device__ inline void finish_pair(const GemmArgs& a, long t, int slab, int q, f32x4 lo, f32x4 hi) {
    auto store_bf16 = [&](long col, f32x4 v) {
        *(u32x2*)((bf16_t*)a.out + t * a.ldo + col) = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
    };
    const long c0 = a.col + slab + 4 * q;
    if constexpr (EPI == JH_EPI_ROPE_BF16) {
        if (slab < a.rope_cols) {
            const long ps = (long)(a.pos[t] & 0xffff) * 32 + 4 * q;
            const f32x4 c = *(const f32x4*)(a.cos_t + ps), sn = *(const f32x4*)(a.sin_t + ps);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float l = lo[e], h = hi[e];
                rope_rotate(l, h, c[e], sn[e]);
                lo[e] = l;
                hi[e] = h;
            }
        }
        store_bf16(c0, lo);
        store_bf16(c0 + 32, hi);
    } else if constexpr (EPI == JH_EPI_GEGLU_BF16) {
        f32x4 g;
#pragma unroll
        for (int e = 0; e < 4; ++e) g[e] = gelu_erf(lo[e]) * hi[e];
        store_bf16(a.col + slab / 2 + 4 * q, g);
    } else {
        finish_one<EPI>(a, t, slab + 4 * q, lo);
        finish_one<EPI>(a, t, slab + 32 + 4 * q, hi);
    }
}

// Small batches in one launch, without the split-K workspace or its reduce
// kernel.  A workgroup owns a BF-feature (64 or 32) x 32-token tile and the
// whole K, resident in LDS as K/64 segments of the main kernel's stage layout
// (so the fragment reads are the same conflict-free ones): 144 KB at most, so
// K <= 768 for 64-feature tiles and K <= 1152 for 32-feature tiles.  Each
// segment's DMA is split evenly over the four waves and issued SMALL_DEPTH
// segments ahead; after a per-segment wait and barrier all four waves
// multiply it, wave w the 16-deep slice 4g + w, so the MFMAs run while later
// segments are still arriving (measured on MI355X at 128 tokens: the whole-K
// fetch of a 64x32 tile takes ~3 us with the weights cold in L2, against
// ~1.2 us of MFMA and LDS reads).  The four partial tiles are summed through
// LDS in wave order (deterministic) by all four waves, 8 tokens each, which
// then apply the epilogue.
//
// LayerNorm prologue (LN_EPL > 0, hidden = 64 * LN_EPL = K): X comes from
// FP32 rows.  Each wave loads its 8 rows after the first W segments are
// issued, normalises them as layer_norm_kernel does (same code, same bits)
// and writes the bf16 rows into the X segments; the first segment's barrier
// publishes them.  This replaces a LayerNorm launch between a residual GEMM
// and the next GEMM.
constexpr int SMALL_LDS = 96 * 768;  // bf16 elements of operand LDS per workgroup (144 KB)
constexpr int SMALL_BT = 32;
constexpr int SMALL_DEPTH = 6;  // K segments in flight ahead of the one being multiplied
template <int BF>
constexpr int small_kmax() {
    return SMALL_LDS / (BF + SMALL_BT) / 64 * 64;
}

// s_waitcnt vmcnt(N): all but this wave's N most recent vector-memory
// operations (loads, DMA or stores) have completed.
template <int N>
__device__ inline void vmcnt() {
    static_assert(N >= 0 && N <= 63, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt vmcnt(n * PW), n in [0, SMALL_DEPTH]: all but this wave's DMA of
// its last n issued segments (PW instructions each) has landed.
template <int PW>
__device__ inline void wait_segments(int n) {
    static_assert(SMALL_DEPTH == 6 && PW * SMALL_DEPTH <= 63, "vmcnt range");
    switch (n) {
        case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
        case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PW) : "memory"); break;
        case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * PW) : "memory"); break;
        case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * PW) : "memory"); break;
        case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * PW) : "memory"); break;
        case 5: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * PW) : "memory"); break;
        default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 * PW) : "memory"); break;
    }
}

template <int EPI, bool GATHER, int BF, int LN_EPL, int KSEG = 0>
__global__ __launch_bounds__(256) void gemm_small_kernel(GemmArgs a) {
    constexpr int BT = SMALL_BT, FB = BF / 32, NCH = BF / 4;
    constexpr bool LNX = LN_EPL > 0;
    // K/64 when known at compile time (the prologue's hidden size, or the
    // instance's K): the segment loop is then unrolled with every wait count an
    // immediate, which at two MFMAs per wave per segment is measurably faster
    // than the loop with a computed wait.
    constexpr int CSEG = LNX ? LN_EPL : KSEG;
    constexpr int WI = BF / 8, XI = LNX ? 0 : BT / 8;  // DMA instructions (8 rows x 128 B) per K segment
    constexpr int PW = (WI + XI) / 4;                  // ... per wave
    static_assert((WI + XI) % 4 == 0 && (BF == 64 || BF == 32), "tile shape");
    static_assert(!LNX || (BF == 64 && !GATHER), "LayerNorm prologue: 64-feature tiles, contiguous rows");
    __shared__ __align__(1024) bf16_t smem[SMALL_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nF = a.n / BF;
    const int f0 = (int)(blockIdx.x % nF) * BF, t0 = (int)(blockIdx.x / nF) * BT;
    const int nseg = CSEG ? CSEG : a.k / 64;  // 128-byte row segments
    bf16_t* const sW = smem;                   // segment g: rows [0, BF) at sW + g*BF*64
    bf16_t* const sX = smem + nseg * BF * 64;  // segment g: rows [0, BT) at sX + g*BT*64
    const i32x4 rw = make_rsrc(a.w + (long)f0 * a.k, (uint64_t)BF * a.k * 2);
    const i32x4 rx = LNX ? i32x4{0, 0, 0, 0}
                         : make_rsrc(a.x + (long)t0 * a.ldx, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)a.k * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

    // Segment g: instructions [0, WI) bring W rows 8j .. 8j+7, [WI, WI+XI) X
    // rows; wave w issues instructions w*PW .. w*PW+PW-1.  Token rows past the
    // end are clamped (their products are never stored).
    auto issue = [&](int g) {
        const uint32_t kb = (uint32_t)g * 128;
#pragma unroll
        for (int u = 0; u < PW; ++u) {
            const int j = wave * PW + u;  // wave-uniform
            if (j < WI) {
                const int row = j * 8 + (lane >> 3);
                const uint32_t l = __builtin_amdgcn_readfirstlane(lds0 + (uint32_t)((g * BF + j * 8) * 64) * 2);
                const uint32_t off = (uint32_t)(row * a.k + (((lane & 7) ^ swz(row)) * 8)) * 2;
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(l), "v"(off), "s"(rw), "s"(kb)
                             : "memory");
            } else if constexpr (XI > 0) {
                const int row = (j - WI) * 8 + (lane >> 3), c = (lane & 7) ^ swz(row);
                const uint32_t l = __builtin_amdgcn_readfirstlane(
                    lds0 + (uint32_t)((nseg * BF * 64 + (g * BT + (j - WI) * 8) * 64) * 2));
                const int t = min(t0 + row, a.rows - 1);
                if constexpr (GATHER) {
                    const bf16_t* src = a.x + (long)a.gather[t] * a.ldx + g * 64 + c * 8;
                    asm volatile("global_load_lds_dwordx4 %1, off" ::"{m0}"(l), "v"(src) : "memory");
                } else {
                    const uint32_t off = (uint32_t)((t - t0) * (long)a.ldx + c * 8) * 2;
                    asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(l), "v"(off), "s"(rx), "s"(kb)
                                 : "memory");
                }
            }
        }
    };

    int issued = min(SMALL_DEPTH, nseg);
    for (int g = 0; g < issued; ++g) issue(g);
    if constexpr (LNX) {
        // Loads complete in issue order, so these rows arrive after the W
        // segments issued above; the compiler's waits for them cover that.
        constexpr int VEC = RowVec<LN_EPL>::VEC;
        RowVec<LN_EPL> xr[8], lw, lb;
#pragma unroll
        for (int r = 0; r < 8; ++r) xr[r].load(a.xf + (long)min(t0 + wave * 8 + r, a.rows - 1) * a.ldx, lane);
        lw.load(a.ln_w, lane);
        if (a.ln_b) lb.load(a.ln_b, lane);
        // RowVec::layer_norm's steps with the 8 rows' reductions interleaved.
        float st[8], mean[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) st[r] = xr[r].sum();
        wave_sum_n(st);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            mean[r] = st[r] * RowVec<LN_EPL>::kInvN;
            st[r] = xr[r].sq_dev(mean[r]);
        }
        wave_sum_n(st);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const int rr = wave * 8 + r;
            xr[r].scale_shift(mean[r], RowVec<LN_EPL>::rstd(st[r], a.ln_eps), lw, a.ln_b ? &lb : nullptr);
#pragma unroll
            for (int c = 0; c < RowVec<LN_EPL>::NC; ++c) {
                const int kk = RowVec<LN_EPL>::index(c, lane), o = kk & 63;
                bf16_t* d = sX + (kk >> 6) * BT * 64 + rr * 64 + (((o >> 3) ^ swz(rr)) * 8) + (o & 7);
                const float* v = xr[r].v + c * VEC;
                if constexpr (VEC == 4) *(u32x2*)d = u32x2{pack2(v[0], v[1]), pack2(v[2], v[3])};
                else if constexpr (VEC == 2) *(uint32_t*)d = pack2(v[0], v[1]);
                else *d = f2bf(v[0]);
            }
        }
    }

    const int lr = lane & 31, lg = lane >> 5, c = wave * 2 + lg;  // chunk pair of slice 4g + wave
    f32x16 acc[FB];
#pragma unroll
    for (int i = 0; i < FB; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.0f;
    auto multiply = [&](int g) {
        const bf16x8 bx = *(const bf16x8*)&sX[g * BT * 64 + lr * 64 + ((c ^ swz(lr)) * 8)];
#pragma unroll
        for (int i = 0; i < FB; ++i) {
            const int r = i * 32 + lr;
            const bf16x8 af = *(const bf16x8*)&sW[g * BF * 64 + r * 64 + ((c ^ swz(r)) * 8)];
            acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bx, acc[i], 0, 0, 0);
        }
    };
    if constexpr (CSEG > 0) {
        constexpr int NSEG = CSEG, ISSUED0 = NSEG < SMALL_DEPTH ? NSEG : SMALL_DEPTH;
        [&]<int... G>(std::integer_sequence<int, G...>) {
            (
                [&] {
                    constexpr int ISSUED = ISSUED0 + G < NSEG ? ISSUED0 + G : NSEG;
                    vmcnt<PW * (ISSUED - G - 1)>();  // this wave's part of segment G has landed
                    __syncthreads();                 // ... and every wave's
                    if constexpr (ISSUED < NSEG) issue(ISSUED);
                    multiply(G);
                }(),
                ...);
        }(std::make_integer_sequence<int, NSEG>{});
    } else {
        for (int g = 0; g < nseg; ++g) {
            wait_segments<PW>(issued - g - 1);  // this wave's part of segment g has landed
            __syncthreads();                     // ... and every wave's
            if (issued < nseg) issue(issued++);
            multiply(g);
        }
    }
    __syncthreads();  // operand LDS is free: reused for the partial tiles
    // Partial tile of wave w: [token][NCH 16-byte chunks of 4 features], the
    // chunk index XOR-swizzled by the token so both passes spread over banks.
    // acc[i][4qd + e] is feature i*32 + qd*8 + 4*lg + e of token lr.
    float* const red = (float*)smem;
    auto slot = [&](int w, int tok, int ch) { return ((w * BT + tok) * NCH + (ch ^ (tok & (NCH - 1)))) * 4; };
#pragma unroll
    for (int i = 0; i < FB; ++i)
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            f32x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[i][qd * 4 + e];
            *(f32x4*)&red[slot(wave, lr, i * 8 + qd * 2 + lg)] = v;
        }
    __syncthreads();
    // Wave w finishes tokens 8w .. 8w+7, lane -> (token 8w + lane/8, chunk q).
    const int tl = wave * 8 + (lane >> 3), q = lane & 7;
    const long t = t0 + tl;
    if (t >= a.rows) return;
    auto total = [&](int ch) {
        f32x4 s = *(const f32x4*)&red[slot(0, tl, ch)];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const f32x4 v = *(const f32x4*)&red[slot(w, tl, ch)];
#pragma unroll
            for (int e = 0; e < 4; ++e) s[e] += v[e];
        }
        return s;
    };
    if constexpr (BF == 64) finish_pair<EPI>(a, t, f0, q, total(q), total(q + 8));
    else finish_one<EPI>(a, t, f0 + 4 * q, total(q));
}

// Split-K reduction + epilogue: thread (row t, 64-wide slab, q) sums the S
// partials of columns slab + 4q .. +3 and slab + 32 + 4q .. +3 in split order
// and applies the same elementwise epilogue, with the same expression order,
// as the GEMM's own epilogue.
template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce(GemmArgs a, int S) {
    const long id = (long)blockIdx.x * 256 + threadIdx.x;
    const int slabs = a.n / 64;
    const long t = id / (slabs * 8);
    if (t >= a.rows) return;
    const int rem = (int)(id - t * slabs * 8), slab = (rem >> 3) * 64, q = rem & 7;
    const size_t plane = (size_t)a.rows * a.n;
    const float* p = a.partial + (size_t)t * a.n + slab + 4 * q;
    // All partial loads first (unconditional: planes past S re-read plane
    // S-1 and are not added), then the sums in split order.
    f32x4 pl[SPLITK_MAX], ph[SPLITK_MAX];
#pragma unroll
    for (int s = 0; s < SPLITK_MAX; ++s) {
        const float* ps = p + (size_t)min(s, S - 1) * plane;
        pl[s] = *(const f32x4*)ps;
        ph[s] = *(const f32x4*)(ps + 32);
    }
    f32x4 lo = pl[0], hi = ph[0];
#pragma unroll
    for (int s = 1; s < SPLITK_MAX; ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo[e] = s < S ? lo[e] + pl[s][e] : lo[e];
            hi[e] = s < S ? hi[e] + ph[s][e] : hi[e];
        }
    finish_pair<EPI>(a, t, slab, q, lo, hi);
}

// Tile shape: 128 features x 128 tokens, four waves of 64x64, two resident
// workgroups per CU (64 KB of LDS each).  Measured on MI355X against 256x128
// (8 waves of 64x64, three 48 KB stages, one workgroup per CU; 384 instead of
// 512 DMA bytes per MFMA) and 256x256 (8 waves of 128x64): in the encoder
// forward they tie at config1 and lose ~10% at M = 16384, because the two
// independent workgroups per CU hide each other's prologue, barrier waits and
// epilogue, which a single workgroup per CU leaves exposed.  A 256x128 tile
// with BK 32, three 24 KB stages and four 128x64 waves keeps two workgroups
// per CU and moves 25% fewer bytes per MFMA (L2 -> LDS and LDS -> registers),
// yet its K loop took as many cycles per MFMA; with the DMA spread between
// the MFMAs it only tied.  In this kernel the shader clock runs at ~1.5-1.8
// GHz (against ~2.2 GHz for the same MFMAs without operand traffic), i.e. the
// GEMMs are power-limited by operand movement as much as by issue.
// Split count for an output of `tiles` 128x128 tiles: enough workgroups to
// cover the GPU about once (256 CUs x 2 resident) when the tile count alone
// leaves most CUs idle, at least two 64-deep K steps per split, and the
// partials must fit the workspace.
int splitk_count(const GemmArgs& a, long tiles) {
    const int kt = a.k / BK;
    if (!a.partial) return 1;
    int s = a.splits > 0 ? a.splits : (tiles >= 128 ? 1 : (int)((384 + tiles - 1) / tiles));
    s = std::min({s, kt / 2, SPLITK_MAX});
    while (s > 1 && (size_t)s * a.rows * a.n * sizeof(float) > a.partial_bytes) --s;
    if (s <= 1) return 1;
    const int chunk = (kt + s - 1) / s;
    return (kt + chunk - 1) / chunk;
}

// Workgroups of gemm_kernel resident at once on the current device (two per
// CU), rounded down to a multiple of 8 XCDs; the persistent kernel's grid.
int resident_tiles() {
    static std::atomic<int> cached[64];
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) throw jh_error(1, "gemm: device ordinal out of range");
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        int cus = 0;
        HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        v = std::max(8, (2 * cus) / 8 * 8);
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Tile width (64 or 32 features) of the one-launch small-batch kernel for
// `a`, or 0 when launch_gemm does not use it.  It replaces split-K where
// split-K would run automatically (workspace given, no forced split count)
// and K fits its LDS; with the LayerNorm prologue it is the only kernel.
// 32-feature tiles move fewer operand bytes per CU, so they are taken when
// their workgroups fit one per CU (then for K up to 1152 as well), for the
// epilogues without a 64-feature pairing.
int small_bf(int epi, const GemmArgs& a) {
    if (a.xf) return 64;
    const long tiles = (long)((a.n + 127) / 128) * ((a.rows + 127) / 128);
    if (!a.partial || a.splits != 0 || splitk_count(a, tiles) <= 1) return 0;
    const bool paired = epi == JH_EPI_ROPE_BF16 || epi == JH_EPI_GEGLU_BF16;
    const long wg32 = (long)(a.n / 32) * ((a.rows + SMALL_BT - 1) / SMALL_BT);
    if (!paired && a.k <= small_kmax<32>() && wg32 <= resident_tiles() / 2) return 32;
    return a.k <= small_kmax<64>() ? 64 : 0;
}

template <int EPI>
void launch_small(const GemmArgs& a, int bf, hipStream_t s) {
    constexpr bool PAIRED = EPI == JH_EPI_ROPE_BF16 || EPI == JH_EPI_GEGLU_BF16;
    const dim3 grid((unsigned)((a.n / bf) * ((a.rows + SMALL_BT - 1) / SMALL_BT))), block(256);
    if (a.xf) {
        if constexpr (PAIRED || EPI == JH_EPI_STORE_BF16) {
            switch (a.k) {
                case 128: JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 2>), grid, block, 0, s, a); break;
                case 256: JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 4>), grid, block, 0, s, a); break;
                case 384: JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 6>), grid, block, 0, s, a); break;
                case 512: JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 8>), grid, block, 0, s, a); break;
                case 768: JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 12>), grid, block, 0, s, a); break;
                default: throw jh_error(1, "gemm: the LayerNorm prologue needs K = hidden in {128, 256, 384, 512, 768}");
            }
        } else {
            throw jh_error(1, "gemm: the LayerNorm prologue supports the STORE, ROPE and GEGLU epilogues");
        }
    } else if (bf == 32) {
        if constexpr (!PAIRED) {
            if (a.gather) JH_LAUNCH((gemm_small_kernel<EPI, true, 32, 0>), grid, block, 0, s, a);
            else if (a.k == 384) JH_LAUNCH((gemm_small_kernel<EPI, false, 32, 0, 6>), grid, block, 0, s, a);
            else if (a.k == 768) JH_LAUNCH((gemm_small_kernel<EPI, false, 32, 0, 12>), grid, block, 0, s, a);
            else if (a.k == 1152) JH_LAUNCH((gemm_small_kernel<EPI, false, 32, 0, 18>), grid, block, 0, s, a);
            else JH_LAUNCH((gemm_small_kernel<EPI, false, 32, 0>), grid, block, 0, s, a);
        } else {
            throw jh_error(1, "gemm: paired epilogues need 64-feature tiles");
        }
    } else {
        if (a.gather) JH_LAUNCH((gemm_small_kernel<EPI, true, 64, 0>), grid, block, 0, s, a);
        else if (a.k == 384) JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 0, 6>), grid, block, 0, s, a);
        else if (a.k == 768) JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 0, 12>), grid, block, 0, s, a);
        else JH_LAUNCH((gemm_small_kernel<EPI, false, 64, 0>), grid, block, 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

// Which kernel launch_gemm runs for `a` (past the small-batch and split-K
// paths) and its tile geometry: BF features x BT tokens per tile, token blocks
// grouped GROUP at a time, `grid` workgroups; for the eight-wave kernel, the
// rows [0, mix) in BT-token tiles and the rest in (BT-32)-token tiles.
struct GemmPlan {
    enum Kind { PLAIN, PERSIST, BIG } kind;
    int bf, bt, group, grid, mix;
};

GemmPlan plan_gemm(const GemmArgs& a) {
    constexpr int BF = 128, BT = 128;
    const int blocks = ((a.n + BF - 1) / BF) * ((a.rows + BT - 1) / BT);
    const int resident = resident_tiles();
    if (a.gather || blocks <= resident) return {GemmPlan::PLAIN, 128, 128, 8, blocks, 0};
    // More tiles than resident workgroups.  Each candidate is costed as its
    // rounds of resident workgroups times the time one round took on
    // MI355X (K = 768, N = 2304, one box): persistent 128x128 12.9 us and
    // 128x192 20.6 us at two workgroups per CU; eight-wave 256x192 19.0
    // and 256x256 22.4 us at one per CU.  A round of eight-wave tiles 32
    // tokens shorter costs ~6% less (the operand DMA, which bounds the K
    // loop, still moves the same W slice per step): 17.9 and 21.1 us.
    auto rounds = [](long tiles, long slots) { return (tiles + slots - 1) / slots; };
    const long t192 = (long)((a.n + 127) / 128) * ((a.rows + 191) / 192);
    const long r128 = rounds(blocks, resident), r192 = rounds(t192, resident);
    // Persistent 128-feature tiles: 192 tokens when their rounds, at 1.5x
    // the work each, cost no more than the 128-token tiles' rounds.
    const bool p192 = t192 >= resident && 3 * r192 <= 2 * r128;
    double best = p192 ? r192 * 20.6 : r128 * 12.9;
    int big = 0;
    long mix = 0;
    if (a.n >= 1024) {
        const int grid = resident / 2;
        const long nF = (a.n + 255) / 256;
        // (256x128 never beats the persistent 128x128 tiles: it has at least
        // their rounds at a higher cost per round.)
        const int bts[2] = {256, 192};
        const double per_round[2] = {22.4, 19.0}, per_short[2] = {21.1, 17.9};
        for (int c = 0; c < 2; ++c) {
            const int bt = bts[c];
            const long nT = (a.rows + bt - 1) / bt;
            const double cost = rounds(nF * nT, grid) * per_round[c];
            if (cost < best) best = cost, big = bt, mix = 0;
            // na full-height token blocks, then the rest in shorter ones, so
            // the second round carries smaller tiles instead of idle CUs
            // (measured for two rounds; more are left uniform).
            for (long na = nT - 1; na >= 1; --na) {
                const long nb = (a.rows - na * bt + bt - 33) / (bt - 32);
                if (nF * na > grid || nF * nb > grid) continue;
                const double cm = per_round[c] + per_short[c];
                if (cm < best) best = cm, big = bt, mix = na * bt;
            }
        }
    }
    if (big) {
        const long nF = (a.n + 255) / 256;
        const long tiles = mix ? nF * std::max(mix / big, (a.rows - mix + big - 33) / (big - 32))
                               : nF * ((a.rows + big - 1) / big);
        return {GemmPlan::BIG, 256, big, 4, (int)std::min<long>(resident / 2, tiles), (int)mix};
    }
    return {GemmPlan::PERSIST, 128, p192 ? 192 : 128, 8, resident, 0};
}

template <int EPI>
void launch_cfg(const GemmArgs& a, hipStream_t s) {
    constexpr int BF = 128, BT = 128;
    const int blocks = ((a.n + BF - 1) / BF) * ((a.rows + BT - 1) / BT);
    if (const int bf = small_bf(EPI, a)) {
        launch_small<EPI>(a, bf, s);
        return;
    }
    const int S = splitk_count(a, blocks);
    if (S > 1) {
        GemmArgs p = a;
        const int kt = a.k / BK;
        p.kt_chunk = (kt + S - 1) / S;
        if (a.gather) JH_LAUNCH((gemm_kernel<EPI_PARTIAL, true>), dim3(blocks * S), dim3(256), 0, s, p);
        else JH_LAUNCH((gemm_kernel<EPI_PARTIAL, false>), dim3(blocks * S), dim3(256), 0, s, p);
        HIP_CHECK(hipGetLastError());
        const long threads = (long)a.rows * (a.n / 64) * 8;
        JH_LAUNCH((splitk_reduce<EPI>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, p, S);
        HIP_CHECK(hipGetLastError());
        return;
    }
    // Weight-stationary kernel whenever W comes packed for it, for every
    // token count: a row's sums then run in one order whatever else is in the
    // batch (the tiled kernels step K by 16, this one by 32, so switching
    // kernels on the batch size would move a row's outputs by FP32 rounding).
    if (gemm_ws_supported(EPI, a)) {
        launch_gemm_ws(EPI, a, s);
        return;
    }
    const GemmPlan pl = plan_gemm(a);
    const dim3 g((unsigned)pl.grid);
    if (pl.kind == GemmPlan::PLAIN) {
        if (a.gather) JH_LAUNCH((gemm_kernel<EPI, true>), g, dim3(256), 0, s, a);
        else JH_LAUNCH((gemm_kernel<EPI, false>), g, dim3(256), 0, s, a);
    } else if (pl.kind == GemmPlan::BIG) {
        GemmArgs b = a;
        b.mix_rows = pl.mix;
        if (pl.bt == 256) JH_LAUNCH((gemm_big_kernel<EPI, 256>), g, dim3(512), 0, s, b);
        else JH_LAUNCH((gemm_big_kernel<EPI, 192>), g, dim3(512), 0, s, b);
    } else if (pl.bt == 192) {
        JH_LAUNCH((gemm_persist_kernel<EPI, 192>), g, dim3(256), 0, s, a);
    } else {
        JH_LAUNCH((gemm_persist_kernel<EPI>), g, dim3(256), 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}

}  // namespace

namespace {

// Shape, alignment and argument checks shared by every GEMM entry; false when
// there is nothing to do (rows == 0).
bool validate_gemm(int epi, const GemmArgs& a) {
    if (a.rows < 0 || a.n <= 0 || a.k <= 0 || a.k % BK || a.n % 64 || a.k > 8192)
        throw jh_error(1, "gemm: need K % 64 == 0, N % 64 == 0, K <= 8192");
    if (a.rows == 0) return false;
    if (a.xf) {
        // LayerNorm prologue: FP32 rows, 16-byte aligned, whole rows of K = hidden.
        if (!a.w || !a.out || !a.ln_w) throw jh_error(1, "gemm: null operand");
        if (a.gather || a.splits)
            throw jh_error(1, "gemm: the LayerNorm prologue takes contiguous rows and no forced split-K");
        if (a.k > small_kmax<64>() || a.ldx % 4 || a.ldx < a.k || ((uintptr_t)a.xf & 15) || ((uintptr_t)a.w & 15))
            throw jh_error(1, "gemm: LayerNorm prologue needs K <= 768, 16-byte aligned rows, ldx % 4 == 0, ldx >= K");
    } else {
        if (!a.x || !a.w || !a.out) throw jh_error(1, "gemm: null operand");
        if (a.ldx % 8 || a.ldx < a.k || ((uintptr_t)a.x & 15) || ((uintptr_t)a.w & 15))
            throw jh_error(1, "gemm: x/w must be 16-byte aligned with ldx % 8 == 0 and ldx >= K");
    }
    const bool f32out = epi == JH_EPI_RESID_F32 || epi == JH_EPI_BIAS_F32;
    const long width = epi == JH_EPI_GEGLU_BF16 ? a.n / 2 : a.n;
    const int per16 = f32out ? 4 : 8;  // elements per 16-byte store
    if (a.col < 0 || a.ldo < a.col + width || a.ldo % per16 || a.col % per16 || ((uintptr_t)a.out & 15))
        throw jh_error(1, "gemm: output columns out of range, or rows/columns not 16-byte aligned");
    const bool needs_bias = epi == JH_EPI_BIAS_BF16 || epi == JH_EPI_BIAS_RELU_BF16 || epi == JH_EPI_BIAS_F32;
    if (needs_bias && !a.bias) throw jh_error(1, "gemm: epilogue needs a bias");
    if (epi == JH_EPI_ROPE_BF16 && a.rope_cols > 0 && (!a.pos || !a.cos_t || !a.sin_t || a.rope_cols % 64))
        throw jh_error(1, "gemm: RoPE epilogue needs pos, cos, sin and rope_cols % 64 == 0");
    if (epi == JH_EPI_GEGLU_BF16 && a.n % 64) throw jh_error(1, "gemm: GEGLU needs N % 64 == 0");
    if (epi < JH_EPI_STORE_BF16 || epi > JH_EPI_BIAS_F32) throw jh_error(1, "gemm: unknown epilogue");
    return true;
}

}  // namespace

bool validate_gemm_args(int epi, const GemmArgs& a) { return validate_gemm(epi, a); }

int gemm_splitk_count(int epi, const GemmArgs& a) {
    if (!validate_gemm(epi, a)) return 1;
    return splitk_count(a, (long)((a.n + 127) / 128) * ((a.rows + 127) / 128));
}

bool gemm_uses_small(int epi, const GemmArgs& a) {
    return validate_gemm(epi, a) && small_bf(epi, a) != 0;
}

void launch_gemm_partial(int epi, const GemmArgs& a, int splits, hipStream_t s) {
    if (!validate_gemm(epi, a)) return;
    if (splits < 2 || !a.partial || (size_t)splits * a.rows * a.n * sizeof(float) > a.partial_bytes ||
        splits > SPLITK_MAX || splits > a.k / BK)
        throw jh_error(1, "gemm: split-K partial pass needs 2..16 splits fitting the workspace");
    GemmArgs p = a;
    const int kt = a.k / BK;
    p.kt_chunk = (kt + splits - 1) / splits;
    if ((kt + p.kt_chunk - 1) / p.kt_chunk != splits) throw jh_error(1, "gemm: split count leaves an empty K chunk");
    const int blocks = ((a.n + 127) / 128) * ((a.rows + 127) / 128);
    if (a.gather) JH_LAUNCH((gemm_kernel<EPI_PARTIAL, true>), dim3(blocks * splits), dim3(256), 0, s, p);
    else JH_LAUNCH((gemm_kernel<EPI_PARTIAL, false>), dim3(blocks * splits), dim3(256), 0, s, p);
    HIP_CHECK(hipGetLastError());
}

void launch_gemm(int epi, const GemmArgs& a, hipStream_t s) {
    if (!validate_gemm(epi, a)) return;
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
