// Weight-stationary BF16 GEMM for gfx950 at K = 768 (the encoder's Wqkv, Wi
// and Wo, and the head's K = 768 projections at full batch).
//
// out = epi(X · Wᵀ) as in gemm.hip, but each workgroup keeps a 256-row slab
// of W resident for its whole life (160 VGPRs per lane and 64 KB of LDS, or,
// for the GEGLU epilogue, 192 VGPRs) and
// streams only X through LDS.  One workgroup per CU, eight waves (two per
// SIMD); wave w owns 32 W rows as two 16-row blocks ("lo" and "hi") × 768 K,
// i.e. 48 A-fragments of v_mfma_f32_16x16x32_bf16, and multiplies them with
// each 16-token X block that lands in LDS: 48 MFMAs per block and wave in two
// independent accumulator chains, each summing K in order.
//
// Why: at K = 768 the tiled kernels are bound by moving both operands from L2
// into LDS (a 256×192 tile needs ~37 B/clk per CU at full MFMA rate and gets
// ~27).  Here only X moves in the loop: each X element is used for 256 W rows,
// 16 B/clk per CU at full MFMA rate, plus the one-time 384 KB W slab per CU.
//
// Layout.  W comes pre-packed (jh_op_pack_ws) so that each wave's fragment
// (slice s, block lo/hi) is one contiguous 1 KB block in A-fragment order
// (lane l: W row l % 16 of the block, K 32s + 8(l/16) .. +8): coalesced
// 16-byte loads.  The slab's 256 rows are the 64-row blocks 4f .. 4f+3 of W;
// wave w takes rows x0 .. x0+15 (lo) and 32+x0 .. 32+x0+15 (hi) of block
// 4f + w/2 (x0 = 16 (w % 2)).  In the 16×16 accumulator layout (lane l: token
// l % 16, rows 4(l/16) .. +3) each lane then holds the RoPE pair (d, d+32) and
// the GEGLU pair (gate, up) of gemm.hip's interleaved Wi in lo[i] and hi[i].
// An X block is 16 tokens × 768 K in 12 stages of [16 rows][128 B], 16-byte
// chunks XOR-swizzled by (row >> 1) & 7 as in gemm.hip (conflict-free B-fragment
// reads).  RoPE cos/sin rows of the block's tokens are gathered into LDS by DMA.
//
// Schedule.  Workgroups are (token range, feature slab) pairs, dealt so that
// the slabs sharing a token range sit on one XCD (X read once per L2).  Per
// 16-token block: one barrier; then every wave runs the block's 48 MFMAs and,
// between them, issues its share of the next block's X DMA (into the other of
// two X slots) and runs the previous block's epilogue from its second set of
// accumulators, so the epilogue's VALU work and stores issue under the MFMAs
// and both waves of a SIMD stay in their MFMA stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <type_traits>

#include "../../include/julia1_hip_ops.h"
#include "kernels.hpp"

namespace {

constexpr int WS_K = 768;
constexpr int WS_S = WS_K / 32;          // 32-deep K slices
constexpr int WS_ROWS = 256;             // W rows per workgroup
constexpr int WS_TB = 16;                // tokens per block
constexpr int WS_XSLOT = WS_TB * WS_K;   // bf16 elements per X slot (24 KB)
constexpr int WS_NCS = 3;                // cos/sin and position slots (RoPE)
constexpr int WS_CSLOT = WS_TB * 32;     // floats per cos (or sin) slot

__device__ constexpr int swz(int r) { return (r >> 1) & 7; }

template <int EPI>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_ws_kernel(GemmArgs a, int nF,
                                                                                               int R, int nTB) {
    constexpr bool ROPE = EPI == JH_EPI_ROPE_BF16;
    constexpr bool GEGLU = EPI == JH_EPI_GEGLU_BF16;
    constexpr bool F32OUT = EPI == JH_EPI_RESID_F32 || EPI == JH_EPI_BIAS_F32;
    constexpr bool BIASED = EPI == JH_EPI_BIAS_BF16 || EPI == JH_EPI_BIAS_RELU_BF16 || EPI == JH_EPI_BIAS_F32;
    // The last WS_SL slices' fragments stay in LDS where the epilogue needs
    // the registers; GEGLU's fits all 24 slices in VGPRs (and, with fewer
    // B-fragment reads in flight, its own temporaries).
    constexpr int WS_SL = GEGLU ? 0 : 4;
    constexpr int WS_SR = WS_S - WS_SL;   // slices whose fragments are held in VGPRs
    constexpr int WS_PD = GEGLU ? 3 : 6;  // B-fragment reads in flight
    __shared__ __align__(1024) bf16_t sx[2 * WS_XSLOT];
    __shared__ __align__(1024) bf16_t swl[WS_SL ? 8 * WS_SL * 2 * 512 : 8];  // each wave's LDS-held fragments
    __shared__ __align__(16) float scs[ROPE ? WS_NCS * 2 * WS_CSLOT : 4];
    __shared__ __align__(16) int spos[ROPE ? WS_NCS * 64 : 4];   // token metadata of a block, DMA'd
    constexpr bool RESID = EPI == JH_EPI_RESID_F32;
    __shared__ __align__(16) f32x4 sold[RESID ? 8 : 1][2][64];   // [wave][lo/hi][lane]: residual rows, by DMA
    // [wave][lo/hi][lane]: the bias values of the lane's columns, by DMA in the prologue (a register load in
    // the epilogue would wait, with vmcnt(0), for the X DMA issued before it)
    __shared__ __align__(16) f32x4 sbias[BIASED || RESID ? 8 : 1][2][64];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // Workgroup -> (token range r, slab f): consecutive ids u share r, and an
    // XCD (workgroup b runs on XCD b % 8) gets a contiguous run of u.
    const int G = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, q8 = G >> 3, r8 = G & 7;
    const int u = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    const int r = u / nF, f = u - r * nF;
    const int b0 = (int)((long)r * nTB / R), b1 = (int)((long)(r + 1) * nTB / R);
    if (b0 >= b1) return;

    // X DMA: instruction i of a block (0..23) fills stage i/2, rows
    // 8(i%2) .. +7; wave w issues i = w, w+8, w+16 (one row half), lane j row
    // 8(w%2) + j/8, the 16-byte chunk that belongs in slot j % 8.  Blocks past
    // the range get an empty resource: their loads read zeros into a slot
    // nothing reads, which keeps the issue branch-free.
    const int drow = 8 * (wave & 1) + (lane >> 3);
    const uint32_t dchunk = (uint32_t)(((lane & 7) ^ swz(drow)) * 16);
    const uint32_t xoff = (uint32_t)drow * (uint32_t)a.ldx * 2 + dchunk;
    auto x_rsrc = [&](int bb) {
        const int t0 = bb * WS_TB;
        return bb < b1 ? make_rsrc(a.x + (long)t0 * a.ldx, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)WS_K * 2)
                       : make_rsrc(a.x, 0);
    };
    auto issue_x = [&](const i32x4& rx, int slot, int j) {  // j-th of this wave's three
        const int i = wave + 8 * j;
        const uint32_t m0 = __builtin_amdgcn_readfirstlane(
            (uint32_t)(uintptr_t)&sx[slot * WS_XSLOT + (i >> 1) * 1024 + (i & 1) * 512]);
        asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(xoff), "s"(rx), "s"((i >> 1) * 128)
                     : "memory");
    };
    // RoPE: the cos and sin rows of the block's tokens, row i at [i][32]
    // (16-byte chunks swizzled as the X rows), at the positions that
    // issue_pos brought into LDS a block earlier.  (Positions go through LDS
    // because a register load would make the compiler wait for it, and vmcnt
    // completes in order: that wait would also wait for every DMA and W load
    // issued before it.)  Waves 0-3 issue one instruction each (cos or sin,
    // rows 0-7 or 8-15); only slabs with rotated rows need the tables.
    const bool rot_slab = ROPE && WS_ROWS * f < a.rope_cols;
    auto issue_pos = [&](int bb, int slot) {  // wave 0: tok_meta of tokens bb·16 .. (64 lanes)
        if constexpr (ROPE) {
            if (rot_slab && wave == 0) {
                const int t0 = bb * WS_TB;
                const i32x4 rp = bb < b1 ? make_rsrc(a.pos + t0, (uint64_t)(a.rows - t0) * 4) : make_rsrc(a.pos, 0);
                const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&spos[slot * 64]);
                asm volatile("buffer_load_dword %1, %2, %3 offen lds" ::"{m0}"(m0), "v"((uint32_t)lane * 4),
                             "s"(rp), "s"(0)
                             : "memory");
            }
        }
    };
    auto issue_cs = [&](int bb, int slot) {
        if constexpr (ROPE) {
            if (rot_slab && wave < 4) {
                const int p = spos[slot * 64 + drow] & 0xffff;
                const float* tab = (wave & 2) ? a.sin_t : a.cos_t;
                const i32x4 rt = make_rsrc(tab, bb < b1 ? 65536ull * 128 : 0);
                const uint32_t m0 = __builtin_amdgcn_readfirstlane(
                    (uint32_t)(uintptr_t)&scs[(2 * slot + (wave >> 1)) * WS_CSLOT + (wave & 1) * 256]);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"((uint32_t)p * 128 + dchunk),
                             "s"(rt), "s"(0)
                             : "memory");
            }
        }
    };

    // Prologue.  The first block's X (and the positions of the first two
    // blocks) ahead of every W load in the CU's queue; then every wave's W
    // fragments: slices 0 .. WS_SR-1 into VGPRs (in K order, pinned: the
    // scheduler otherwise reorders them and the first MFMA waits for nearly
    // all of them; they land in order and the first block's MFMAs wait for
    // each in turn), the rest by DMA into this wave's LDS fragments.
    const bool two = b0 + 1 < b1;
    {
        const i32x4 rx = x_rsrc(b0);
#pragma unroll
        for (int j = 0; j < 3; ++j) issue_x(rx, 0, j);
        issue_pos(b0, 0);
        if (two) issue_pos(b0 + 1, 1);
        if constexpr (BIASED || RESID) {
            if (a.bias) {
                const int bcol = 64 * (4 * f + (wave >> 1)) + 16 * (wave & 1) + 4 * (lane >> 4);
                const i32x4 rb = make_rsrc(a.bias, (uint64_t)a.n * 4);
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbias[wave][h][0]);
                    asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"((uint32_t)bcol * 4),
                                 "s"(rb), "s"(h * 128)
                                 : "memory");
                }
            }
        }
    }
    __syncthreads();
    bf16x8 wf[WS_SR][2];
    const bf16_t* wp = a.w_ws + (long)(f * 8 + wave) * WS_S * 2 * 512;
#pragma unroll
    for (int s = 0; s < WS_SR; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            wf[s][h] = *(const bf16x8*)(wp + (s * 2 + h) * 512 + lane * 8);
            __builtin_amdgcn_sched_barrier(0);
        }
    if constexpr (WS_SL > 0) {
        const i32x4 rw = make_rsrc(wp + WS_SR * 2 * 512, WS_SL * 2 * 1024);
#pragma unroll
        for (int j = 0; j < WS_SL * 2; ++j) {
            const uint32_t m0 =
                __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&swl[(wave * WS_SL * 2 + j) * 512]);
            asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"((uint32_t)lane * 16), "s"(rw),
                         "s"(j * 1024)
                         : "memory");
        }
    }
    // the first block's X, positions and bias landed (48 W loads and DMAs since)
    asm volatile("s_waitcnt vmcnt(48)" ::: "memory");
    __syncthreads();

    const int tk = lane & 15, kg = lane >> 4;  // B-fragment token, K group; accumulator rows 4·kg ..
    const int hb = 4 * f + (wave >> 1), x0 = 16 * (wave & 1);
    const bf16_t* WL = swl + wave * WS_SL * 2 * 512 + lane * 8;
    f32x4 acc[2][2];  // [set][lo/hi]

    // Epilogue of block bb from accumulator set P: lane (tk, kg) holds token
    // bb·16 + tk, columns x0 + 4kg .. +3 of the lo half (acc[P][0]) and of the
    // hi half (acc[P][1]).  Split into steps so the block loop can spread
    // them between its MFMAs.  Lanes l, l+16, l+32, l+48 write one token's 32
    // contiguous bytes per half.
    struct EpiState {
        f32x4 lo, hi, c, sn;
        int t;
    };
    auto epi_begin = [&](EpiState& e, int P, int bb) {
        e.t = bb * WS_TB + tk;
        e.lo = acc[P][0];
        e.hi = acc[P][1];
    };
    // Step j (0..4) of the elementwise part: j = 0 loads what the others
    // need (cos/sin rows from LDS, bias), j = 1..4 finish column i = j - 1,
    // so the VALU work spreads over five MFMA slices.
    auto epi_step = [&](EpiState& e, int j, int cslot) {
        if constexpr (ROPE) {
            if (hb * 64 < a.rope_cols) {
                if (j == 0) {
                    const float* C = scs + (2 * cslot) * WS_CSLOT;
                    const float* S = C + WS_CSLOT;
                    const int ch = (((x0 >> 2) + kg) ^ swz(tk)) * 4;
                    e.c = *(const f32x4*)&C[tk * 32 + ch];
                    e.sn = *(const f32x4*)&S[tk * 32 + ch];
                } else {
                    float l = e.lo[j - 1], h = e.hi[j - 1];
                    rope_rotate(l, h, e.c[j - 1], e.sn[j - 1]);
                    e.lo[j - 1] = l;
                    e.hi[j - 1] = h;
                }
            }
        }
        if constexpr (GEGLU) {
            if (j > 0) e.lo[j - 1] = gelu_erf(e.lo[j - 1]) * e.hi[j - 1];
        }
        if constexpr (BIASED) {
            if (j == 0) {
                e.c = sbias[wave][0][lane];
                e.sn = sbias[wave][1][lane];
            } else {
                e.lo[j - 1] += e.c[j - 1];
                e.hi[j - 1] += e.sn[j - 1];
                if constexpr (EPI == JH_EPI_BIAS_RELU_BF16) {
                    e.lo[j - 1] = fmaxf(e.lo[j - 1], 0.0f);
                    e.hi[j - 1] = fmaxf(e.hi[j - 1], 0.0f);
                }
            }
        }
    };
    auto epi_math = [&](EpiState& e, int cslot) {
#pragma unroll
        for (int j = 0; j < 5; ++j) epi_step(e, j, cslot);
    };
    // The stores go through a buffer resource that ends at the block's last
    // token, so the range check drops rows past it and no branch is needed:
    // behind a branch, the compiler sinks the elementwise steps into it, to
    // the end of the block, away from the MFMA slices they are spread over.
    auto epi_store = [&](EpiState& e) {
        constexpr int ESZ = F32OUT ? 4 : 2;
        const int t0 = e.t - tk, nt = a.rows - t0 < WS_TB ? a.rows - t0 : WS_TB;
        const int col = a.col + (GEGLU ? 32 : 64) * hb + x0 + 4 * kg;
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
            (char*)a.out + (long)t0 * a.ldo * ESZ, 0, nt * a.ldo * ESZ, 0x00020000);
        const int vo = (tk * a.ldo + col) * ESZ;
        if constexpr (GEGLU) {
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2(e.lo[0], e.lo[1]), pack2(e.lo[2], e.lo[3])}, ro, vo,
                                                  0, 0);
        } else if constexpr (F32OUT) {
            if constexpr (EPI == JH_EPI_RESID_F32) {
                // the residual rows, DMA'd into LDS a block ahead (issue_old)
                const f32x4 olo = sold[wave][0][lane], ohi = sold[wave][1][lane];
                f32x4 lo = e.lo, hi = e.hi;
                if (a.bias) {
                    const f32x4 b_lo = sbias[wave][0][lane], b_hi = sbias[wave][1][lane];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        lo[i] += b_lo[i];
                        hi[i] += b_hi[i];
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    lo[i] = olo[i] + lo[i];
                    hi[i] = ohi[i] + hi[i];
                }
                __builtin_amdgcn_raw_buffer_store_b128(lo, ro, vo, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(hi, ro, vo + 32 * ESZ, 0, 0);
            } else {
                __builtin_amdgcn_raw_buffer_store_b128(e.lo, ro, vo, 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(e.hi, ro, vo + 32 * ESZ, 0, 0);
            }
        } else {
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2(e.lo[0], e.lo[1]), pack2(e.lo[2], e.lo[3])}, ro, vo, 0,
                                                  0);
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{pack2(e.hi[0], e.hi[1]), pack2(e.hi[2], e.hi[3])}, ro,
                                                  vo + 32 * ESZ, 0, 0);
        }
    };

    // RESID: the residual values a wave's lanes add to (block bb, its 16
    // tokens, columns col .. +3 and col + 32 .. +3) are DMA'd into LDS at the
    // end of the block, a block ahead of the epilogue that adds them, which
    // waits for them with an explicit count: a register load would make the
    // compiler wait with vmcnt(0), and vmcnt completes in order, so that wait
    // would also wait for the X DMA issued since.  Rows past the last token
    // read zeros (their sums are dropped by the store's range check).
    auto issue_old = [&](int bb) {
        if constexpr (RESID) {
            const int t0 = bb * WS_TB, nt = a.rows - t0 < WS_TB ? a.rows - t0 : WS_TB;
            const int col = a.col + 64 * hb + x0 + 4 * kg;
            const i32x4 ro = make_rsrc((const float*)a.out + (long)t0 * a.ldo, (uint64_t)nt * a.ldo * 4);
            const uint32_t vo = (uint32_t)(tk * a.ldo + col) * 4;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sold[wave][h][0]);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(vo), "s"(ro), "s"(h * 128)
                             : "memory");
            }
        }
    };

    // One block bb into accumulator set P from X slot (bb - b0) % 2.  Between
    // the MFMAs: the next block's X DMA (after slices 1, 3, 5), its RoPE rows
    // (7) and the positions of the block after (9), and, with EPI_PREV, the
    // previous block's epilogue from set 1-P (elementwise steps after slices
    // 10-14, stores after 16: the last VMEM instructions of the block).  FIRST: block b0,
    // whose W fragments are still landing (the compiler waits for each before
    // its MFMA) and whose LDS-held fragments must have landed before they are
    // read; it also gathers its own RoPE rows.
    auto block = [&](auto PC, auto EPI_PREV, auto FIRST, int bb) {
        constexpr int P = decltype(PC)::value;
        const int k = bb - b0;
        const bf16_t* X = sx + (k & 1) * WS_XSLOT;
        auto rd = [&](int s) {
            const int c = (s & 1) * 4 + kg;
            return *(const bf16x8*)&X[(s >> 1) * 1024 + tk * 64 + ((c ^ swz(tk)) * 8)];
        };
        const i32x4 rx = x_rsrc(bb + 1);
        EpiState e;
        if constexpr (decltype(EPI_PREV)::value) epi_begin(e, 1 - P, bb - 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[P][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        bf16x8 bx[WS_PD], wl[2][2];
#pragma unroll
        for (int p = 0; p < WS_PD; ++p) bx[p] = rd(p);
#pragma unroll
        for (int s = 0; s < WS_S; ++s) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bf16x8 w = s < WS_SR ? wf[s < WS_SR ? s : 0][h] : wl[(s - WS_SR) & 1][h];
                acc[P][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w, bx[s % WS_PD], acc[P][h], 0, 0, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (s + WS_PD < WS_S) bx[s % WS_PD] = rd(s + WS_PD);
            if (WS_SL > 0 && s >= WS_SR - 2 && s < WS_S - 2) {  // LDS-held fragments of slice s + 2 (two buffers)
                if (decltype(FIRST)::value && s == WS_SR - 2) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                const int sl = s + 2 - WS_SR;
#pragma unroll
                for (int h = 0; h < 2; ++h) wl[sl & 1][h] = *(const bf16x8*)&WL[(sl * 2 + h) * 512];
            }
            if (s == 1 || s == 3 || s == 5) issue_x(rx, (k + 1) & 1, s >> 1);
            if (s == 7) {
                if (decltype(FIRST)::value) issue_cs(b0, 0);
                issue_cs(bb + 1, (k + 1) % WS_NCS);
            }
            if (s == 9) issue_pos(bb + 2, (k + 2) % WS_NCS);
            if constexpr (decltype(EPI_PREV)::value) {
                if (s >= 10 && s < 15) epi_step(e, s - 10, (k - 1) % WS_NCS);
                if (s == 16) {
                    // RESID: the residual rows landed (the 3 X DMA instructions since may not have)
                    if constexpr (RESID) asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
                    epi_store(e);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        issue_old(bb);
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using T = std::true_type;
    using F = std::false_type;

    // Each block starts with a barrier (its X, RoPE rows and positions
    // landed; the slots of two blocks back are free), for which each wave
    // waits for its own DMA, but not for the stores of the epilogue it ran
    // since: those are its last VMEM instructions, 2 of them (1 for GEGLU),
    // issued whether or not their rows are past the last token; with RESID
    // the two residual-row DMAs of issue_old follow them (and, in the first
    // block, come alone).
    auto sync = [&](int k) {
        if constexpr (RESID) {
            if (k == 1) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        } else {
            if (k == 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            else if constexpr (GEGLU) asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        }
        __syncthreads();
    };
    block(C0{}, F{}, T{}, b0);
    int bb = b0 + 1;
    for (; bb + 1 < b1; bb += 2) {
        sync(bb - b0);
        block(C1{}, T{}, F{}, bb);
        sync(bb + 1 - b0);
        block(C0{}, T{}, F{}, bb + 1);
    }
    if (bb < b1) {
        sync(bb - b0);
        block(C1{}, T{}, F{}, bb);
    }
    // The last block's epilogue (its RoPE rows landed at its own barrier,
    // except for a single-block range, whose rows were issued in its block).
    if (b1 == b0 + 1) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    EpiState e;
    const int kl = b1 - 1 - b0;
    if (kl & 1) epi_begin(e, 1, b1 - 1);
    else epi_begin(e, 0, b1 - 1);
    epi_math(e, kl % WS_NCS);
    if constexpr (RESID) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // its residual rows
    epi_store(e);
}

// K-split weight-stationary kernel for K = 1152 (the MLP-out projection Wo2,
// out f32 += X · Wᵀ (+ bias)).  A 256-row slab of K = 1152 (576 KB) does not
// fit a CU's registers, so each workgroup keeps a 128-row slab and splits K
// between partner waves: wave w holds rows 32·(w % 4) .. +31 (two 16-row
// groups, "lo" and "hi") for K slices 18·(w / 4) .. +17, 144 VGPRs.  Per
// 16-token block each wave runs 36 MFMAs over its half of K (each X fragment
// feeding both row groups); the upper-half waves (w ≥ 4) leave their sums in
// LDS at the end of the block, and during the next block the lower-half
// partner adds them to its own (lower half + upper half, in that order) and
// runs the residual epilogue.  X streams through two LDS slots as in
// gemm_ws_kernel (18 stages of [16 rows][128 B] per block, DMA issued by all
// eight waves between their MFMAs).
constexpr int W2_K = 1152;
constexpr int W2_ROWS = 128;             // W rows per workgroup
constexpr int W2_PD = 6;                 // B-fragment reads in flight

template <int KS>  // 32-deep K slices
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_ws2_kernel(GemmArgs a, int nF,
                                                                                                int R, int nTB) {
    constexpr int W2_K = KS * 32;
    constexpr int W2_SH = KS / 2;            // slices per K half
    constexpr int W2_XSLOT = WS_TB * W2_K;   // bf16 elements per X slot
    constexpr int W2_XI = W2_K / 64 * 2;     // 1 KB X DMA instructions per block
    constexpr int W2_NXL = (W2_XI - 4) / 8 + 1;  // of which a lower-half wave (w < 4) issues
    constexpr int W2_ES = W2_SH - 4;         // slice after which the previous block's epilogue runs
    __shared__ __align__(1024) bf16_t sx[2 * W2_XSLOT];
    __shared__ __align__(16) f32x4 spart[2][4][2][64];  // [block parity][row group][lo/hi][lane]
    __shared__ __align__(16) f32x4 sold[4][2][64];      // [row group][lo/hi][lane]: residual rows, by DMA
    __shared__ __align__(16) f32x4 sbias[4][2][64];     // [row group][lo/hi][lane]: bias, by DMA in the prologue

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int rg = wave & 3, kh = wave >> 2;
    const int G = gridDim.x, bid = blockIdx.x;
    const int xcd = bid & 7, local = bid >> 3, q8 = G >> 3, r8 = G & 7;
    const int u = xcd * q8 + (xcd < r8 ? xcd : r8) + local;
    const int r = u / nF, f = u - r * nF;
    const int b0 = (int)((long)r * nTB / R), b1 = (int)((long)(r + 1) * nTB / R);
    if (b0 >= b1) return;

    // X DMA: instruction i (0 .. 35) fills stage i / 2, rows 8(i % 2) .. +7;
    // wave w issues i = w, w + 8, ... (i % 2 == w % 2), lane j row 8(w % 2) + j / 8.
    const int drow = 8 * (wave & 1) + (lane >> 3);
    const uint32_t dchunk = (uint32_t)(((lane & 7) ^ swz(drow)) * 16);
    const uint32_t xoff = (uint32_t)drow * (uint32_t)a.ldx * 2 + dchunk;
    auto x_rsrc = [&](int bb) {
        const int t0 = bb * WS_TB;
        return bb < b1 ? make_rsrc(a.x + (long)t0 * a.ldx, (uint64_t)(a.rows - 1 - t0) * a.ldx * 2 + (uint64_t)W2_K * 2)
                       : make_rsrc(a.x, 0);
    };
    auto issue_x = [&](const i32x4& rx, int slot, int j) {
        const int i = wave + 8 * j;
        if (i < W2_XI) {
            const uint32_t m0 = __builtin_amdgcn_readfirstlane(
                (uint32_t)(uintptr_t)&sx[slot * W2_XSLOT + (i >> 1) * 1024 + (i & 1) * 512]);
            asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(xoff), "s"(rx),
                         "s"((i >> 1) * 128)
                         : "memory");
        }
    };

    // Prologue: the first block's X ahead of every W load, then this wave's
    // 36 W fragments in K order (pinned, so the first MFMAs wait for each in turn).
    {
        const i32x4 rx = x_rsrc(b0);
#pragma unroll
        for (int j = 0; j < 5; ++j) issue_x(rx, 0, j);
        if (a.bias && kh == 0) {
            const i32x4 rb = make_rsrc(a.bias, (uint64_t)a.n * 4);
            const uint32_t bo = (uint32_t)(W2_ROWS * f + 32 * rg + 4 * (lane >> 4)) * 4;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sbias[rg][h][0]);
                asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(bo), "s"(rb), "s"(h * 64)
                             : "memory");
            }
        }
    }
    __syncthreads();
    bf16x8 wf[W2_SH][2];
    const bf16_t* wp = a.w_ws + (long)(f * 8 + wave) * W2_SH * 2 * 512;
#pragma unroll
    for (int s = 0; s < W2_SH; ++s)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            wf[s][h] = *(const bf16x8*)(wp + (s * 2 + h) * 512 + lane * 8);
            __builtin_amdgcn_sched_barrier(0);
        }
    // the first block's X and the bias landed (the 36 W loads issued since may not have)
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * W2_SH) : "memory");
    __syncthreads();

    const int tk = lane & 15, kg = lane >> 4;
    const int col = a.col + W2_ROWS * f + 32 * rg + 4 * kg;  // lo columns; hi = col + 16
    f32x4 acc[2][2];                                          // [set][lo/hi]

    // The residual values a lower-half wave's lanes add to (block bb, its 16
    // tokens, columns col .. +3 and col + 16 .. +3) are DMA'd into LDS at the
    // end of the block, a block ahead of the epilogue that adds them; its wait
    // for them is an explicit count (a register load would make the compiler
    // wait with vmcnt(0), and vmcnt completes in order: that wait would also
    // wait for the X DMA issued since).  Rows past the last token read zeros.
    auto issue_old = [&](int bb) {
        const int t0 = bb * WS_TB, nt = a.rows - t0 < WS_TB ? a.rows - t0 : WS_TB;
        const i32x4 ro = make_rsrc((const float*)a.out + (long)t0 * a.ldo, (uint64_t)nt * a.ldo * 4);
        const uint32_t vo = (uint32_t)(tk * a.ldo + col) * 4;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)&sold[rg][h][0]);
            asm volatile("buffer_load_dwordx4 %1, %2, %3 offen lds" ::"{m0}"(m0), "v"(vo), "s"(ro), "s"(h * 64)
                         : "memory");
        }
    };
    // Residual epilogue of block bb from accumulator set P (lower-half waves,
    // its residual rows landed in LDS): sum = own + partner's (LDS), + bias,
    // out = old + sum, through a buffer resource ending at the block's last
    // token (rows past it are dropped).
    auto epilogue = [&](int P, int bb) {
        const int t0 = bb * WS_TB, nt = a.rows - t0 < WS_TB ? a.rows - t0 : WS_TB;
        const f32x4 plo = spart[(bb - b0) & 1][rg][0][lane], phi = spart[(bb - b0) & 1][rg][1][lane];
        const f32x4 olo = sold[rg][0][lane], ohi = sold[rg][1][lane];
        f32x4 lo, hi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = acc[P][0][i] + plo[i];
            hi[i] = acc[P][1][i] + phi[i];
        }
        if (a.bias) {
            const f32x4 b_lo = sbias[rg][0][lane], b_hi = sbias[rg][1][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[i] += b_lo[i];
                hi[i] += b_hi[i];
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = olo[i] + lo[i];
            hi[i] = ohi[i] + hi[i];
        }
        const __amdgpu_buffer_rsrc_t ro =
            __builtin_amdgcn_make_buffer_rsrc((char*)a.out + (long)t0 * a.ldo * 4, 0, nt * a.ldo * 4, 0x00020000);
        const int vo = (tk * a.ldo + col) * 4;
        __builtin_amdgcn_raw_buffer_store_b128(lo, ro, vo, 0, 0);
        __builtin_amdgcn_raw_buffer_store_b128(hi, ro, vo + 64, 0, 0);
    };

    // One block bb into accumulator set P from X slot (bb - b0) % 2: the
    // next block's X DMA after slices 1, 3, .., 9 (five instructions for a
    // lower-half wave); with EPI_PREV the lower-half waves run the previous
    // block's epilogue after slice 14, once its residual rows (DMA'd before
    // those five) landed.  At the end the upper-half waves leave this block's
    // sums in LDS and the lower-half waves issue its residual-row DMA.
    auto block = [&](auto PC, auto EPI_PREV, int bb) {
        constexpr int P = decltype(PC)::value;
        const int k = bb - b0;
        const bf16_t* X = sx + (k & 1) * W2_XSLOT;
        auto rd = [&](int s) {
            const int gs = W2_SH * kh + s, c = (gs & 1) * 4 + kg;
            return *(const bf16x8*)&X[(gs >> 1) * 1024 + tk * 64 + ((c ^ swz(tk)) * 8)];
        };
        const i32x4 rx = x_rsrc(bb + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[P][h] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        bf16x8 bx[W2_PD];
#pragma unroll
        for (int p = 0; p < W2_PD; ++p) bx[p] = rd(p);
#pragma unroll
        for (int s = 0; s < W2_SH; ++s) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int h = 0; h < 2; ++h)
                acc[P][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wf[s][h], bx[s % W2_PD], acc[P][h], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (s + W2_PD < W2_SH) bx[s % W2_PD] = rd(s + W2_PD);
            if (s == 1 || s == 3 || s == 5 || s == 7 || s == 9) issue_x(rx, (k + 1) & 1, s >> 1);
            if constexpr (decltype(EPI_PREV)::value) {
                if (s == W2_ES && kh == 0) {
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(W2_NXL) : "memory");
                    epilogue(1 - P, bb - 1);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        if (kh == 1) {
            spart[k & 1][rg][0][lane] = acc[P][0];
            spart[k & 1][rg][1][lane] = acc[P][1];
        } else {
            issue_old(bb);
        }
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    using T = std::true_type;
    using F = std::false_type;

    // Each block starts with a barrier: its X landed (each wave waits for its
    // own DMA, but a lower-half wave not for its last VMEM instructions: the
    // two stores of its epilogue, none in the first block, and the two
    // residual-row DMAs after them), the previous block's upper-half sums are
    // in LDS, and the slots of two blocks back are free.
    auto sync = [&](int k) {
        if (kh == 1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if (k == 1) asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        __syncthreads();
    };
    block(C0{}, F{}, b0);
    int bb = b0 + 1;
    for (; bb + 1 < b1; bb += 2) {
        sync(bb - b0);
        block(C1{}, T{}, bb);
        sync(bb + 1 - b0);
        block(C0{}, T{}, bb + 1);
    }
    if (bb < b1) {
        sync(bb - b0);
        block(C1{}, T{}, bb);
    }
    // the last block's upper-half sums and residual rows
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kh == 0) {
        if ((b1 - 1 - b0) & 1) epilogue(1, b1 - 1);
        else epilogue(0, b1 - 1);
    }
}

int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) throw jh_error(1, "gemm: device ordinal out of range");
    int v = cached[dev].load(std::memory_order_relaxed);
    if (v == 0) {
        HIP_CHECK(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
        v = std::max(v, 1);
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

}  // namespace

bool gemm_ws_supported(int epi, const GemmArgs& a) {
    if (!a.w_ws || a.gather || a.xf || a.rows <= 0 || ((uintptr_t)a.w_ws & 15)) return false;
    if (a.k == W2_K) return a.n % W2_ROWS == 0 && epi == JH_EPI_RESID_F32;
    return a.k == WS_K && a.n % WS_ROWS == 0 && epi >= JH_EPI_STORE_BF16 && epi <= JH_EPI_BIAS_F32;
}

// W rows per workgroup of the kernel that takes K.
static int ws_rows(int k) { return k == W2_K ? W2_ROWS : WS_ROWS; }

// Token ranges per slab: as many as fill the CUs (at most one block each).
int gemm_ws_ranges(const GemmArgs& a) {
    const int nF = a.n / ws_rows(a.k), nTB = (a.rows + WS_TB - 1) / WS_TB;
    return std::max(1, std::min(nTB, device_cus() / nF));
}

int gemm_ws_block_tokens() { return WS_TB; }

void launch_gemm_ws(int epi, const GemmArgs& a, hipStream_t s) {
    if (!gemm_ws_supported(epi, a))
        throw jh_error(1, "gemm: weight-stationary kernel needs packed W and K = 768 with N % 256 == 0, or K = 1152 "
                          "with N % 128 == 0 and the residual epilogue");
    const int nF = a.n / ws_rows(a.k), nTB = (a.rows + WS_TB - 1) / WS_TB, R = gemm_ws_ranges(a);
    const dim3 grid((unsigned)(nF * R)), block(512);
    if (a.k == W2_K) {
        JH_LAUNCH((gemm_ws2_kernel<W2_K / 32>), grid, block, 0, s, a, nF, R, nTB);
        HIP_CHECK(hipGetLastError());
        return;
    }
    switch (epi) {
        case JH_EPI_STORE_BF16: JH_LAUNCH((gemm_ws_kernel<JH_EPI_STORE_BF16>), grid, block, 0, s, a, nF, R, nTB); break;
        case JH_EPI_ROPE_BF16: JH_LAUNCH((gemm_ws_kernel<JH_EPI_ROPE_BF16>), grid, block, 0, s, a, nF, R, nTB); break;
        case JH_EPI_GEGLU_BF16: JH_LAUNCH((gemm_ws_kernel<JH_EPI_GEGLU_BF16>), grid, block, 0, s, a, nF, R, nTB); break;
        case JH_EPI_RESID_F32: JH_LAUNCH((gemm_ws_kernel<JH_EPI_RESID_F32>), grid, block, 0, s, a, nF, R, nTB); break;
        case JH_EPI_BIAS_BF16: JH_LAUNCH((gemm_ws_kernel<JH_EPI_BIAS_BF16>), grid, block, 0, s, a, nF, R, nTB); break;
        case JH_EPI_BIAS_RELU_BF16:
            JH_LAUNCH((gemm_ws_kernel<JH_EPI_BIAS_RELU_BF16>), grid, block, 0, s, a, nF, R, nTB);
            break;
        case JH_EPI_BIAS_F32: JH_LAUNCH((gemm_ws_kernel<JH_EPI_BIAS_F32>), grid, block, 0, s, a, nF, R, nTB); break;
        default: throw jh_error(1, "gemm: unknown epilogue");
    }
    HIP_CHECK(hipGetLastError());
}

// Host-side packing of a bf16 [n, k] row-major W into the weight-stationary
// fragment order: [slab f][wave w][slice s][lo/hi h][lane l][8], lane l
// holding W row 64(4f + w/2) + 32h + 16(w % 2) + l % 16, K 32s + 8(l/16) .. +8.
// At K = 1152 (the K-split kernel): 128-row slabs, lane l of wave w holding W
// row 128f + 32(w % 4) + 16h + l % 16, K 32(18(w / 4) + s) + 8(l/16) .. +8.
void pack_ws(const bf16_t* w, int n, int k, bf16_t* out) {
    if (k == W2_K) {
        const int W2_SH = k / 64;
        for (int f = 0; f < n / W2_ROWS; ++f)
            for (int wave = 0; wave < 8; ++wave)
                for (int s = 0; s < W2_SH; ++s)
                    for (int h = 0; h < 2; ++h)
                        for (int lane = 0; lane < 64; ++lane) {
                            const int rw = W2_ROWS * f + 32 * (wave % 4) + 16 * h + lane % 16;
                            bf16_t* o = out + (((((long)f * 8 + wave) * W2_SH + s) * 2 + h) * 64 + lane) * 8;
                            const bf16_t* src = w + (long)rw * k + 32 * (W2_SH * (wave / 4) + s) + 8 * (lane / 16);
                            for (int e = 0; e < 8; ++e) o[e] = src[e];
                        }
        return;
    }
    const int ns = k / 32;
    for (int f = 0; f < n / WS_ROWS; ++f)
        for (int wave = 0; wave < 8; ++wave)
            for (int s = 0; s < ns; ++s)
                for (int h = 0; h < 2; ++h)
                    for (int lane = 0; lane < 64; ++lane) {
                        const int rw = 64 * (4 * f + wave / 2) + 32 * h + 16 * (wave % 2) + lane % 16;
                        bf16_t* o = out + (((((long)f * 8 + wave) * ns + s) * 2 + h) * 64 + lane) * 8;
                        const bf16_t* src = w + (long)rw * k + 32 * s + 8 * (lane / 16);
                        for (int e = 0; e < 8; ++e) o[e] = src[e];
                    }
}
