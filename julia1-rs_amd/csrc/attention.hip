// FlashAttention-2 forward for gfx950: one workgroup of four waves per
// (128-query tile, head); each wave owns 32 queries.  Four waves share every
// staged K/Vᵀ tile (half the LDS staging per query of a 64-query tile), and
// the register budget is held to four resident waves per SIMD (at most 128
// VGPRs) so that one wave's softmax VALU work (more than its MFMA time at
// head_dim 64) overlaps other waves' MFMAs.  Measured on MI355X at L = 8192:
// 1.6x the throughput of two-wave workgroups at two waves per SIMD.
//
// The score tile is computed transposed, Sᵀ = K·Qᵀ, with
// v_mfma_f32_32x32x16_bf16 (M = 32 keys, N = 32 queries, K = 16 head dims).
// The accumulator layout then gives every lane ONE query (column l%32) and
// 16 of its keys, the other 16 sitting in lane l^32 — so the online-softmax
// state (running max m, running sum l) is one scalar per lane and each row
// reduction is a single cross-half exchange.  The output is also produced
// transposed, Oᵀ = Vᵀ·Pᵀ: Pᵀ as the MFMA B operand needs, per lane, that same
// query and 8 keys, which are exactly 8 of the Sᵀ accumulator values the lane
// already holds (the MFMA's K order is a permutation of keys; Vᵀ is read in
// the same permutation).  P therefore never leaves registers.
//
// K and V tiles (64 keys x 64 dims) reach LDS by buffer DMA, row-major with
// 128-byte key rows and XOR-swizzled 16-byte chunks, double buffered (the DMA
// of tile it+1 runs under the math of tile it).  K fragments are 16-byte
// reads of key rows.  The Vᵀ fragments of Oᵀ = Vᵀ·Pᵀ come from gfx950's
// transposing LDS read ds_read_b64_tr_b16 (measured lane layout: in each
// group of 16 lanes, output lane i, element k' is element i%4 of the 4
// bf16 that source lane 4k' + i/4 addresses): source lane j pointing at
// V[kb + j/4][d0 + 4(j%4)] gives output lane i the 4 keys kb..kb+3 of dim
// d0 + i.  No register staging or VALU transpose of V remains.
// Sliding-window tiles only visit keys in [q_pos - window, q_pos + nq - 1 +
// window] ∩ [0, kv_len), with per-element masking of |q - k| <= window.
//
// Per 64-key tile a wave issues 16 MFMAs (512 cycles of its SIMD's MFMA pipe)
// against ~150 other VALU instructions, 32 of them v_exp_f32 (~8 cycles each
// on gfx950, the others 2-5); measured, MFMA and VALU time largely add up at
// head_dim 64, so the softmax is kept lean: the running max is only moved,
// and O rescaled, when it grows by more than 2^11 in p (a wave-uniform
// branch), which removes most of the 32 rescale multiplies per tile.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "kernels.hpp"

namespace {

constexpr int KT = 64;       // keys per LDS tile
// Lazy rescale threshold of the slow path (log2 units: it keeps p <= 2^11),
// and the bound on a lane's sum of its 32 p values under which the fast path
// keeps a tile.  The sum bounds each p, so a kept tile has every p <= 2^16:
// up to 2^5 above the slow path's bound, and still far inside what bf16 P,
// the FP32 row sums and the FP32 O accumulators carry without overflow or
// loss of relative precision.
constexpr float kLazyLog2 = 11.0f;
constexpr float kSumMax = 65536.0f;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

// Chunk swizzles of the 128-byte key rows.  K: 32 consecutive rows read one
// 16-byte chunk each (as the GEMM operands).  V: a half-wave's transposing
// reads touch 4 consecutive rows x 4 chunks; rows r and r+2 share a bank half,
// so their chunks are moved 4 apart.
__device__ constexpr int kswz(int r) { return (r >> 1) & 7; }
__device__ constexpr int vswz(int r) { return ((r >> 1) & 1) << 2; }

// NW waves per workgroup, 32 queries each: 4 (128-query tiles) everywhere, or
// 8 (256-query tiles) for the global layers of long sequences, where each
// staged K/V tile then serves twice the queries (global layer at 4 x 8192:
// 2% faster; slower for sequences of ~1k tokens and for window layers).  The
// eight-wave form stages two key tiles per barrier (four 16 KB K/V slots,
// 64 KB: two workgroups per CU still fit), which halves the barriers each
// wave meets (a further 1.8% at 4 x 8192).
template <int NW, bool WIN>  // WIN: a window layer (a.window >= 0), whose tiles run one 32-key block per step
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(4))) void attention_kernel(AttnArgs a) {
    constexpr int SPB = NW / 4;           // key tiles staged per barrier
    constexpr int RPW = SPB * KT / NW;    // K/V rows each wave stages per barrier (8 per DMA instruction)
    __shared__ __align__(1024) bf16_t sK[2 * SPB][KT * 64];
    __shared__ __align__(1024) bf16_t sV[2 * SPB][KT * 64];

    // One workgroup per (tile, head), heads varying fastest: callers list the
    // costliest tiles first, so those are dispatched first, one per CU.
    const int head = (int)(blockIdx.x % (unsigned)a.heads);
    const AttnTile tile = a.tiles[blockIdx.x / (unsigned)a.heads];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 31, g = lane >> 5;

    const bf16_t* kbase = a.k + (long)tile.kv_row * a.ldkv + head * 64;
    const bf16_t* vbase = a.v + (long)tile.kv_row * a.ldkv + head * 64;

    // Q fragments (B operand of Sᵀ = K·Qᵀ): query lq of this wave, dims ks*16 + 8g .. +7.
    const int qi = wave * 32 + lq;  // query index within the tile
    bf16x8 qf[4];
    {
        const bool ok = qi < tile.nq;
        const bf16_t* qp = a.q + (long)(tile.q_row + (ok ? qi : 0)) * a.ldq + head * 64 + g * 8;
        u32x4 r[4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) r[ks] = ok ? *(const u32x4*)(qp + ks * 16) : u32x4{0, 0, 0, 0};
        // Consume the loaded registers here, so the compiler waits for these
        // loads once, before the key loop.  Otherwise its wait for them sits
        // in front of every tile's first MFMA as vmcnt(0), which also waits
        // out the next tile's K/V DMA issued just before it.
        asm volatile("" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) qf[ks] = __builtin_bit_cast(bf16x8, r[ks]);
    }
    const int qpos = tile.q_pos + qi;

    int kbeg = 0, kend = tile.kv_len;
    if (a.window >= 0) {
        kbeg = max(0, tile.q_pos - a.window);
        kend = min(tile.kv_len, tile.q_pos + tile.nq + a.window);
    }

    // DMA of one stage (SPB K/V tiles, SPB·64 key rows) into stage buffer
    // `st`: wave w fills rows [RPW·w, RPW·w+RPW) of the stage in both K and V
    // with RPW/8 1 KB instructions each; lane i of instruction j takes row
    // RPW·w + 8j + i/8, physical slot i%8 (the swizzles depend on the row
    // modulo 16, so a row's place inside its 64-row tile decides them).  The lane's byte offsets are
    // fixed per row (the tile adds k0 rows); rows past the sequence end fall
    // outside the buffer resource's range and read as zeros (they are masked
    // to -inf before the softmax, and their zero V rows contribute nothing).
    const i32x4 rsk = make_rsrc(kbase, ((uint64_t)(tile.kv_len - 1) * a.ldkv + 64) * 2);
    const i32x4 rsv = make_rsrc(vbase, ((uint64_t)(tile.kv_len - 1) * a.ldkv + 64) * 2);
    const uint32_t lk0 = (uint32_t)(uintptr_t)&sK[0][0], lv0 = (uint32_t)(uintptr_t)&sV[0][0];
    uint32_t okb[RPW / 8], ovb[RPW / 8];
#pragma unroll
    for (int j = 0; j < RPW / 8; ++j) {
        const int row = RPW * wave + 8 * j + (lane >> 3);
        okb[j] = (uint32_t)(row * a.ldkv + (((lane & 7) ^ kswz(row)) * 8)) * 2;
        ovb[j] = (uint32_t)(row * a.ldkv + (((lane & 7) ^ vswz(row)) * 8)) * 2;
    }
    auto issue = [&](int k0, int st) {
        const uint32_t kt = (uint32_t)(k0 * a.ldkv) * 2;  // bytes of the stage's first key row
#pragma unroll
        for (int j = 0; j < RPW / 8; ++j) {
            const int r0 = RPW * wave + 8 * j;
            const uint32_t lk = __builtin_amdgcn_readfirstlane(lk0 + (st * SPB * KT * 64 + r0 * 64) * 2);
            const uint32_t lv = __builtin_amdgcn_readfirstlane(lv0 + (st * SPB * KT * 64 + r0 * 64) * 2);
            asm volatile("buffer_load_dwordx4 %1, %2, 0 offen lds" ::"{m0}"(lk), "v"(okb[j] + kt), "s"(rsk)
                         : "memory");
            asm volatile("buffer_load_dwordx4 %1, %2, 0 offen lds" ::"{m0}"(lv), "v"(ovb[j] + kt), "s"(rsv)
                         : "memory");
        }
    };
    // Transposing V reads: this lane's 16-lane group G and index j select
    // key row offset 4(G/2) + j/4 and dims 16(G%2) + 4(j%4) .. +3.
    // The row's swizzle vswz(row) equals vswz(vrow) (32kb + 16hb + 8·half keep
    // bit 1), so per dim block db the lane's byte offset inside a tile is fixed;
    // kb, hb and the +8-key half become immediate offsets.
    const int tg = lane >> 4, tj = lane & 15;
    const int vrow = 4 * (tg >> 1) + (tj >> 2);  // + 32kb + 16hb + 8·half
    const int vch = 2 * (tg & 1) + ((tj & 3) >> 1);  // + 4db (16-byte chunk within the 64-dim row)
    const uint32_t voff0 = vrow * 128 + ((vch) ^ vswz(vrow)) * 16 + (tj & 1) * 8;
    const uint32_t voff1 = vrow * 128 + ((4 + vch) ^ vswz(vrow)) * 16 + (tj & 1) * 8;

    f32x16 o[2];
#pragma unroll
    for (int e = 0; e < 16; ++e) o[0][e] = o[1][e] = 0.0f;
    // Online softmax in log2 units: p = exp2(c·s - c·m) with c = scale·log2(e),
    // evaluated as one FMA per score; m is the running max of the raw scores.
    float m = -INFINITY, l = 0.0f;
    const float c = a.scale_log2;
    const float thr = kLazyLog2 / c;  // raw-score growth of the max that forces a rescale
    bool ref_ok = false;              // every lane of the wave has a finite running max
    // Queries of this wave sit at positions [qlo, qlo + 31].
    const int qlo = tile.q_pos + wave * 32;

    const int ntk = kend > kbeg ? (kend - kbeg + KT - 1) / KT : 0;
    if (ntk > 0) issue(kbeg, 0);
    // A wave with no queries in the tile, or whose 32 queries are all outside
    // the window of a key tile, skips that tile's math (uniform per wave); it
    // still stages its share of K/V and meets every barrier.
    const bool active = wave * 32 < tile.nq;
    for (int it = 0; it < ntk; ++it) {
        const int buf = it % (2 * SPB), k0 = kbeg + it * KT;
        // at a stage's first tile: the stage landed (this wave's DMA, then
        // everyone's), and every wave is done with the previous stage, whose
        // buffer the next DMA refills
        if (it % SPB == 0) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (it + SPB < ntk) issue(k0 + SPB * KT, ((it / SPB) + 1) & 1);
        }
        const bool skip = !active || (a.window >= 0 && (k0 > qlo + 31 + a.window || k0 + KT - 1 < qlo - a.window));
        if (skip) continue;
        lds_u8* const vt = (lds_u8*)&sV[buf][0];  // this tile's V buffer
        // One softmax step over NB 32-key blocks of the tile from block kb0:
        // the whole tile (NB = 2), or on window layers each block that holds
        // keys inside the wave's window on its own (NB = 1), which skips the
        // sixth of a wave's blocks that lie wholly outside it.
        auto step = [&](auto NBc, const int kb0) {
        constexpr int NB = decltype(NBc)::value;
        const int kk0 = k0 + 32 * kb0;  // first key of the step

        // Sᵀ for keys [k0, k0+64): two 32-key blocks.
        auto scores = [&](f32x16(&s)[NB]) {
#pragma unroll
            for (int kb = 0; kb < NB; ++kb) {
#pragma unroll
                for (int e = 0; e < 16; ++e) s[kb][e] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int r = (kb0 + kb) * 32 + lq;
                    bf16x8 kf = *(const bf16x8*)&sK[buf][r * 64 + (((ks * 2 + g) ^ kswz(r)) * 8)];
                    s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb], 0, 0, 0);
                }
            }
        };
        // P = exp2(c·s - c·m) rounded to bf16, packed in pairs: pp[kb*8 + w]
        // holds elements 2w, 2w+1 of block kb.  The row sum adds the FP32
        // values in four independent chains.  (v_dot2c_f32_bf16 over the packed
        // pairs would need half the instructions, but on gfx950 it does not
        // issue while an MFMA runs on the SIMD: measured ~7 cycles of MFMA
        // time lost per dot2c, against none for v_add_f32.)
        uint32_t pp[8 * NB];
        float ls = 0.0f;
        auto exps = [&](const f32x16(&s)[NB], float mc) {
            float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int w = 0; w < 8; ++w) {
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][2 * w], c, -mc));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][2 * w + 1], c, -mc));
                    pp[kb * 8 + w] = pack2(p0, p1);
                    part[w & 3] += p0 + p1;
                }
            ls = (part[0] + part[1]) + (part[2] + part[3]);
        };
        // Masking is only needed where this wave's (query, key) block can hold
        // an invalid pair (decided per wave, so the branch is uniform): the
        // sequence end, or a sliding window edge.  Masked scores become -inf,
        // so their p = exp2(-inf) = 0 on either path.
        const bool tail = kk0 + 32 * NB > kend;
        const bool edge = a.window >= 0 && (kk0 < qlo + 31 - a.window || kk0 + 32 * NB - 1 > qlo + a.window);
        auto mask = [&](f32x16(&s)[NB]) {
            // Element e of block kb is key k0 + kb*32 + (e/4)*8 + 4g + e%4;
            // element offset off (key kl + off) is valid iff lo <= off <= hi:
            // off < kend - kl, and |qpos - kl - off| <= window when windowed.
            const int kl = kk0 + 4 * g;  // key of element 0 in block 0 of the step for this lane
            int lo = 0, hi = kend - kl - 1;
            if (a.window >= 0) {
                lo = max(lo, qpos - kl - a.window);
                hi = min(hi, qpos - kl + a.window);
            }
            // Empty range: move lo far right so off - lo wraps to a huge value.
            const unsigned span = hi >= lo ? (unsigned)(hi - lo) : 0u;
            lo = hi >= lo ? lo : 0x40000000;
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int off = kb * 32 + (e >> 2) * 8 + (e & 3);
                    const bool ok = (unsigned)(off - lo) <= span;
                    s[kb][e] = ok ? s[kb][e] : -INFINITY;
                }
        };
        // Fast path: every lane holding a finite running max (masked tiles
        // included).  The max of the tile is then not computed at all: a
        // lane's sum of p bounds each of its p, so a sum within kSumMax = 2^16
        // proves no p exceeded 2^16.  Otherwise (a rare tile whose scores rose
        // far past the running max) the tile is redone on the slow path, which
        // moves the max.
        bool fast = ref_ok;
        if (fast) {
            f32x16 s[NB];
            scores(s);
            if (tail || edge) mask(s);
            exps(s, m * c);
            fast = __builtin_amdgcn_ballot_w64(!(ls <= kSumMax)) == 0;
        }
        if (!fast) {
            f32x16 s[NB];
            scores(s);
            if (tail || edge) mask(s);
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < NB; ++kb)
#pragma unroll
                for (int e = 0; e < 16; ++e) mx = fmaxf(mx, s[kb][e]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            // Lazy rescale: the running max moves (and O, l are rescaled) only
            // when some lane's tile max exceeds it by more than kLazyLog2 in
            // log2 units; the branch is wave-uniform.  Until then p may reach
            // 2^kLazyLog2, which bf16 P and the FP32 sums carry without loss of
            // relative precision, and a lane's 32 values sum to at most kSumMax.
            if (__builtin_amdgcn_ballot_w64(mx > m + thr) != 0) {
                const float mn = fmaxf(m, mx);
                const float alpha = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - mn) * c);
                l *= alpha;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    o[0][e] *= alpha;
                    o[1][e] *= alpha;
                }
                m = mn;
            }
            exps(s, m == -INFINITY ? 0.0f : m * c);
            ref_ok = __builtin_amdgcn_ballot_w64(m == -INFINITY) == 0;
        }
        l += ls;
        // Oᵀ += Vᵀ·Pᵀ over 4 steps of 16 keys.  Step (kb, hb) uses accumulator
        // elements hb*8 .. hb*8+7 of block kb: keys base + 8*(e/4) + 4g + e%4.
#pragma unroll
        for (int kb = 0; kb < NB; ++kb)
#pragma unroll
            for (int hb = 0; hb < 2; ++hb) {
                const bf16x8 pf = __builtin_bit_cast(
                    bf16x8, u32x4{pp[kb * 8 + hb * 4], pp[kb * 8 + hb * 4 + 1], pp[kb * 8 + hb * 4 + 2],
                                  pp[kb * 8 + hb * 4 + 3]});
#pragma unroll
                for (int db = 0; db < 2; ++db) {
                    // keys kb*32 + hb*16 + 4g + (0..3) and + 8 + (0..3) of dim db*32 + lq
                    const int at = (int)(db ? voff1 : voff0) + (kb0 + kb) * 4096 + hb * 2048;
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vt + at));
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(vt + at + 1024));
                    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
                    const bf16x8 vf = __builtin_bit_cast(bf16x8, u32x4{l2[0], l2[1], h2[0], h2[1]});
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, o[db], 0, 0, 0);
                }
            }
        };
        if constexpr (WIN) {
#pragma unroll
            for (int kb0 = 0; kb0 < 2; ++kb0) {
                const int kk0 = k0 + 32 * kb0;
                if (kk0 > qlo + 31 + a.window || kk0 + 31 < qlo - a.window) continue;
                step(std::integral_constant<int, 1>{}, kb0);
            }
        } else {
            step(std::integral_constant<int, 2>{}, 0);
        }
    }

    l += __shfl_xor(l, 32, 64);
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    if (qi < tile.nq) {
        bf16_t* op = a.out + (long)(tile.q_row + qi) * a.ldo + head * 64;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int qd = 0; qd < 4; ++qd) {
                int d = db * 32 + qd * 8 + g * 4;
                *(u32x2*)(op + d) = u32x2{pack2(o[db][qd * 4] * inv, o[db][qd * 4 + 1] * inv),
                                          pack2(o[db][qd * 4 + 2] * inv, o[db][qd * 4 + 3] * inv)};
            }
    }
}

}  // namespace

void launch_attention(const AttnArgs& a, hipStream_t s) {
    if (a.ntiles < 0 || a.heads <= 0) throw jh_error(1, "attention: bad tile/head count");
    if (a.waves != 4 && a.waves != 8) throw jh_error(1, "attention: 4 or 8 waves (128- or 256-query tiles)");
    if (a.ntiles == 0) return;
    if (!a.q || !a.k || !a.v || !a.out || !a.tiles) throw jh_error(1, "attention: null operand");
    if (a.ldq % 8 || a.ldkv % 8 || a.ldo % 4 || a.ldq < a.heads * 64 || a.ldo < a.heads * 64 ||
        ((uintptr_t)a.q & 15) || ((uintptr_t)a.k & 15) || ((uintptr_t)a.v & 15) || ((uintptr_t)a.out & 7))
        throw jh_error(1, "attention: operands must be 16-byte aligned with row strides % 8 == 0");
    if ((long)a.ntiles * a.heads > 0x7fffffffL) throw jh_error(1, "attention: grid too large");
    const dim3 grid((unsigned)(a.ntiles * a.heads));
    if (a.waves == 8) {
        if (a.window >= 0) JH_LAUNCH((attention_kernel<8, true>), grid, dim3(512), 0, s, a);
        else JH_LAUNCH((attention_kernel<8, false>), grid, dim3(512), 0, s, a);
    } else {
        if (a.window >= 0) JH_LAUNCH((attention_kernel<4, true>), grid, dim3(256), 0, s, a);
        else JH_LAUNCH((attention_kernel<4, false>), grid, dim3(256), 0, s, a);
    }
    HIP_CHECK(hipGetLastError());
}
