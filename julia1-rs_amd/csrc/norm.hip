// Row kernels for gfx950: one 64-lane wavefront per row (two for LayerNorm),
// four waves per 256-thread workgroup.  A row of `hidden` floats is held as hidden/64
// values per lane, loaded with the widest vector that divides them (float4
// for hidden 768/1024, float2 for 384/128), so every global access is a fully
// coalesced 64-lane vector load.  LayerNorm is two-pass (mean, then squared
// deviations) with wavefront-shuffle sums, as in the reference's layer_norm.
#include <hip/hip_runtime.h>

#include "kernels.hpp"
#include "rowvec.hpp"

namespace {

constexpr int ROWS_PER_BLOCK = 4;

// First row of this workgroup when the rows are dealt to the 8 XCDs in
// contiguous eighths (workgroup b runs on XCD b % 8), the way the GEMMs deal
// their token tiles: the residual rows x that a row kernel reads were then
// written by GEMM workgroups on the same XCD and are still in its L2.
// Measured on MI355X (config1, A/B on one box): LayerNorm 0.297 -> 0.264 ms
// per forward against rows striped over the XCDs four at a time.
template <int RPB = ROWS_PER_BLOCK>
__device__ inline int xcd_rows_first() {
    const int nb = (int)gridDim.x, xcd = (int)(blockIdx.x & 7), loc = (int)(blockIdx.x >> 3);
    const int q8 = nb >> 3, r8 = nb & 7;
    return (xcd * q8 + (xcd < r8 ? xcd : r8) + loc) * RPB;
}

template <int EPL>
__global__ __launch_bounds__(256) void embed_ln_kernel(const uint32_t* __restrict__ ids, int rows,
                                                       const float* __restrict__ table, const float* __restrict__ w,
                                                       float eps, float* __restrict__ x, bf16_t* __restrict__ xn) {
    constexpr int H = EPL * 64;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    RowVec<EPL> r;
    r.load(table + (long)ids[row] * H, lane);
    r.layer_norm(w, nullptr, eps, lane);
    r.store(x + (long)row * H, lane);
    r.store_bf16(xn + (long)row * H, lane);
}

// LayerNorm: each wave normalises LN_RPW consecutive rows, their loads (and
// one load of the weights) issued together and their reductions interleaved
// -- RowVec::layer_norm's steps in the same order, so the same bits.  Two
// rows per wave fit config1's 9482 rows in one round of wave slots and halve
// the weight re-reads: 0.6% off the whole forward on MI355X (A/B on one box);
// four per wave was slower.
constexpr int LN_RPW = 2;
template <int EPL>
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* __restrict__ x, int rows,
                                                         const float* __restrict__ w, const float* __restrict__ b,
                                                         float eps, bf16_t* __restrict__ out) {
    constexpr int H = EPL * 64;
    const int row0 = xcd_rows_first<4 * LN_RPW>() + (threadIdx.x >> 6) * LN_RPW, lane = threadIdx.x & 63;
    if (row0 >= rows) return;
    RowVec<EPL> r[LN_RPW], g, bb;
#pragma unroll
    for (int i = 0; i < LN_RPW; ++i) r[i].load(x + (long)min(row0 + i, rows - 1) * H, lane);
    g.load(w, lane);
    if (b) bb.load(b, lane);
    float st[LN_RPW], mean[LN_RPW];
#pragma unroll
    for (int i = 0; i < LN_RPW; ++i) st[i] = r[i].sum();
    wave_sum_n(st);
#pragma unroll
    for (int i = 0; i < LN_RPW; ++i) {
        mean[i] = st[i] * RowVec<EPL>::kInvN;
        st[i] = r[i].sq_dev(mean[i]);
    }
    wave_sum_n(st);
#pragma unroll
    for (int i = 0; i < LN_RPW; ++i) {
        if (row0 + i >= rows) break;
        const float rs = RowVec<EPL>::rstd(st[i], eps);
        if (b) r[i].scale_shift(mean[i], rs, g, &bb);
        else r[i].scale_shift(mean[i], rs, g, nullptr);
        r[i].store_bf16(out + (long)(row0 + i) * H, lane);
    }
}

// Split-K residual GEMM finish fused with the LayerNorm that follows it:
// x[row] += Σ_s partial[s][row] (+ bias), summed in split order exactly as
// the GEMM's own split-K reduction does, then out = bf16(LN(x[row])).
template <int EPL>
__global__ __launch_bounds__(256) void resid_reduce_ln_kernel(const float* __restrict__ partial, int S, long plane,
                                                              const float* __restrict__ bias, float* __restrict__ x,
                                                              int rows, const float* __restrict__ w,
                                                              const float* __restrict__ b, float eps,
                                                              bf16_t* __restrict__ out) {
    constexpr int H = EPL * 64;
    const int row = xcd_rows_first() + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* p = partial + (long)row * H;
    RowVec<EPL> acc;
    acc.load(p, lane);
    // Four planes per round, loaded before they are added (planes past S
    // re-read plane S-1 and are skipped).
    for (int s0 = 1; s0 < S; s0 += 4) {
        RowVec<EPL> t[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) t[u].load(p + (long)min(s0 + u, S - 1) * plane, lane);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc.v[e] = s0 + u < S ? acc.v[e] + t[u].v[e] : acc.v[e];
    }
    if (bias) {
        RowVec<EPL> bb;
        bb.load(bias, lane);
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc.v[e] += bb.v[e];
    }
    RowVec<EPL> r;
    r.load(x + (long)row * H, lane);
#pragma unroll
    for (int e = 0; e < EPL; ++e) r.v[e] += acc.v[e];
    r.store(x + (long)row * H, lane);
    r.layer_norm(w, b, eps, lane);
    r.store_bf16(out + (long)row * H, lane);
}

template <int EPL>
__global__ __launch_bounds__(256) void final_norm_kernel(float* __restrict__ x, int rows, const float* __restrict__ fw,
                                                         const float* __restrict__ type_emb,
                                                         const uint32_t* __restrict__ tok_meta,
                                                         const float* __restrict__ hw, const float* __restrict__ hb,
                                                         float eps, bf16_t* __restrict__ out) {
    constexpr int H = EPL * 64;
    const int row = xcd_rows_first() + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    // Every load is issued before the first reduction: the token's type row
    // (behind its tok_meta word), both norms' weights and the row itself, so a
    // wave waits on one round of memory latency instead of three in a row.
    const uint32_t qt = (tok_meta[row] >> 16) & 0xff;
    RowVec<EPL> r, te, g1, g2, b2;
    float* xr = x + (long)row * H;
    r.load(xr, lane);
    g1.load(fw, lane);
    g2.load(hw, lane);
    if (hb) b2.load(hb, lane);
    te.load(type_emb + (long)qt * H, lane);
    r.layer_norm(g1, nullptr, eps);
#pragma unroll
    for (int e = 0; e < EPL; ++e) r.v[e] += te.v[e];
    r.store(xr, lane);
    r.layer_norm(g2, hb ? &b2 : nullptr, 1e-5f);
    r.store_bf16(out + (long)row * H, lane);
}

template <int EPL>
__global__ __launch_bounds__(256) void gather_kernel(const float* __restrict__ src, const int32_t* __restrict__ idx,
                                                     int rows, float* __restrict__ dst) {
    constexpr int H = EPL * 64;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    RowVec<EPL> r;
    r.load(src + (long)idx[row] * H, lane);
    r.store(dst + (long)row * H, lane);
}

template <int EPL>
__global__ __launch_bounds__(256) void scorer_kernel(const float* __restrict__ z, int rows, const float* __restrict__ w2,
                                                     float b2, float* __restrict__ out) {
    constexpr int H = EPL * 64;
    const int row = blockIdx.x * ROWS_PER_BLOCK + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= rows) return;
    RowVec<EPL> r, w;
    r.load(z + (long)row * H, lane);
    w.load(w2, lane);
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) s += gelu_erf(r.v[e]) * w.v[e];
    s = wave_sum(s);
    if (lane == 0) out[row] = s + b2;
}

// Calls f.template operator()<EPL>() for hidden = 64*EPL in the supported set.
template <class F>
void dispatch_hidden(int hidden, F&& f) {
    switch (hidden) {
        case 64: f.template operator()<1>(); break;
        case 128: f.template operator()<2>(); break;
        case 192: f.template operator()<3>(); break;
        case 256: f.template operator()<4>(); break;
        case 320: f.template operator()<5>(); break;
        case 384: f.template operator()<6>(); break;
        case 448: f.template operator()<7>(); break;
        case 512: f.template operator()<8>(); break;
        case 576: f.template operator()<9>(); break;
        case 640: f.template operator()<10>(); break;
        case 704: f.template operator()<11>(); break;
        case 768: f.template operator()<12>(); break;
        case 832: f.template operator()<13>(); break;
        case 896: f.template operator()<14>(); break;
        case 960: f.template operator()<15>(); break;
        case 1024: f.template operator()<16>(); break;
        default: throw jh_error(1, "row kernels support hidden = 64*k for k in 1..16");
    }
}

inline dim3 row_grid(int rows) { return dim3((rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK); }

}  // namespace

void launch_embed_ln(const uint32_t* ids, int rows, const float* table, const float* w, float eps, int hidden,
                     float* x, bf16_t* xn, hipStream_t s) {
    if (rows <= 0) return;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(embed_ln_kernel<EPL>, row_grid(rows), dim3(256), 0, s, ids, rows, table, w, eps, x, xn);
    });
    HIP_CHECK(hipGetLastError());
}

void launch_layer_norm(const float* x, int rows, const float* w, const float* b, float eps, int hidden, bf16_t* out,
                       hipStream_t s) {
    if (rows <= 0) return;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(layer_norm_kernel<EPL>, dim3((rows + 4 * LN_RPW - 1) / (4 * LN_RPW)), dim3(256), 0, s, x, rows, w,
                  b, eps, out);
    });
    HIP_CHECK(hipGetLastError());
}

void launch_resid_reduce_ln(const float* partial, int splits, int rows, int hidden, const float* bias, float* x,
                            const float* w, const float* b, float eps, bf16_t* out, hipStream_t s) {
    if (rows <= 0) return;
    if (splits < 1) throw jh_error(1, "resid_reduce_ln: splits >= 1");
    const long plane = (long)rows * hidden;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(resid_reduce_ln_kernel<EPL>, row_grid(rows), dim3(256), 0, s, partial, splits, plane, bias, x, rows,
                  w, b, eps, out);
    });
    HIP_CHECK(hipGetLastError());
}

void launch_final_norm(float* x, int rows, const float* fw, const float* type_emb, const uint32_t* tok_meta,
                       const float* hw, const float* hb, float eps, int hidden, bf16_t* out, hipStream_t s) {
    if (rows <= 0) return;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(final_norm_kernel<EPL>, row_grid(rows), dim3(256), 0, s, x, rows, fw, type_emb, tok_meta,
                           hw, hb, eps, out);
    });
    HIP_CHECK(hipGetLastError());
}

void launch_gather_f32(const float* src, const int32_t* idx, int rows, int hidden, float* dst, hipStream_t s) {
    if (rows <= 0) return;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(gather_kernel<EPL>, row_grid(rows), dim3(256), 0, s, src, idx, rows, dst);
    });
    HIP_CHECK(hipGetLastError());
}

void launch_scorer(const float* z, int rows, int hidden, const float* w2, float b2, float* out, hipStream_t s) {
    if (rows <= 0) return;
    dispatch_hidden(hidden, [&]<int EPL>() {
        JH_LAUNCH(scorer_kernel<EPL>, row_grid(rows), dim3(256), 0, s, z, rows, w2, b2, out);
    });
    HIP_CHECK(hipGetLastError());
}
