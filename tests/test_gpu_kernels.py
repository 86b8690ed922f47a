"""Kernel-level parity on the GPU: every gfx950 kernel through the C-ABI
(include/julia1_hip_ops.h) against an f64 reference of the same bf16/f32
inputs, and against the FP32 oracle where the oracle has the same op.

Tolerances: bf16 outputs carry one RNE rounding (relative 2^-9), so they are
held to 4e-3 relative; FP32 outputs to 1e-4 of the operand scale (FP32
accumulation-order differences only).
"""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from julia1_amd import abi, hip  # noqa: E402
from oracle import oracle  # noqa: E402
from gpu_util import bf16_round, dev, host  # noqa: E402

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def rng(seed):
    return np.random.default_rng(seed)


def _gemm_inputs(r, rows, n, k):
    x = bf16_round(r.standard_normal((rows, k), dtype=np.float32))
    w = bf16_round(r.standard_normal((n, k), dtype=np.float32) * 0.02)
    return x, w, x.astype(np.float64) @ w.astype(np.float64).T


# The last two have more 128x128 tiles (520) than two per CU on MI355X, so they take the persistent
# kernel (several tiles per workgroup, the next tile's first K step prefetched); K = 64 is its one-step case.
SHAPES = [(1, 64, 64), (37, 128, 768), (130, 384, 1152), (257, 2304, 768), (64, 768, 3072),
          (8300, 1024, 256), (8300, 1024, 64)]


@pytest.mark.parametrize("rows,n,k", SHAPES)
def test_gemm_store_bf16(rows, n, k):
    x, w, ref = _gemm_inputs(rng(1), rows, n, k)
    out = torch.zeros(rows, n + 16, dtype=BF16, device="cuda")
    hip.op_gemm(abi.EPI_STORE_BF16, dev(x, BF16), dev(w, BF16), out, col=8)
    got = host(out)
    assert np.all(got[:, :8] == 0) and np.all(got[:, 8 + n:] == 0)
    d = np.abs(got[:, 8:8 + n] - ref)
    assert np.all(d <= 4e-3 * np.abs(ref) + 1e-6), d.max()


@pytest.mark.parametrize("rows,n,k", SHAPES)
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemm_resid_f32(rows, n, k, with_bias):
    r = rng(2)
    x, w, ref = _gemm_inputs(r, rows, n, k)
    base = r.standard_normal((rows, n), dtype=np.float32)
    bias = r.standard_normal(n, dtype=np.float32) if with_bias else None
    out = dev(base)
    hip.op_gemm(abi.EPI_RESID_F32, dev(x, BF16), dev(w, BF16), out, bias=None if bias is None else dev(bias))
    expect = base + ref + (0 if bias is None else bias)
    assert np.abs(host(out) - expect).max() < 1e-4 * math.sqrt(k) * 0.02 * 4 + 1e-5


@pytest.mark.parametrize("rows,n,k", [(200, 384, 768), (8300, 1024, 128)])
@pytest.mark.parametrize("epi", [abi.EPI_BIAS_BF16, abi.EPI_BIAS_RELU_BF16, abi.EPI_BIAS_F32])
def test_gemm_bias_epilogues(epi, rows, n, k):
    r = rng(3)
    x, w, ref = _gemm_inputs(r, rows, n, k)
    bias = r.standard_normal(n, dtype=np.float32) * 0.1
    dt = torch.float32 if epi == abi.EPI_BIAS_F32 else BF16
    out = torch.zeros(rows, n, dtype=dt, device="cuda")
    hip.op_gemm(epi, dev(x, BF16), dev(w, BF16), out, bias=dev(bias))
    expect = ref + bias
    if epi == abi.EPI_BIAS_RELU_BF16:
        expect = np.maximum(expect, 0)
    tol = 1e-5 if epi == abi.EPI_BIAS_F32 else 4e-3 * np.abs(expect) + 1e-6
    assert np.all(np.abs(host(out) - expect) <= tol)


def test_gemm_gather_rows():
    r = rng(4)
    x, w, ref = _gemm_inputs(r, 300, 256, 512)
    idx = np.array([5, 0, 299, 17, 17, 100, 3], dtype=np.int32)
    out = torch.zeros(idx.size, 256, dtype=torch.float32, device="cuda")
    bias = np.zeros(256, dtype=np.float32)
    hip.op_gemm(abi.EPI_BIAS_F32, dev(x, BF16), dev(w, BF16), out, rows=idx.size, gather=dev(idx), bias=dev(bias))
    assert np.abs(host(out) - ref[idx]).max() < 1e-5


@pytest.mark.parametrize("rows,inter,k", [(1, 64, 128), (77, 192, 128), (300, 1152, 768), (8300, 512, 128)])
def test_gemm_geglu(rows, inter, k):
    r = rng(5)
    x = bf16_round(r.standard_normal((rows, k), dtype=np.float32))
    wi = bf16_round(r.standard_normal((2 * inter, k), dtype=np.float32) * 0.05)
    prod = x.astype(np.float64) @ wi.astype(np.float64).T
    u, v = prod[:, :inter], prod[:, inter:]
    erf = np.vectorize(math.erf)
    expect = 0.5 * u * (1 + erf(u / math.sqrt(2))) * v
    out = torch.zeros(rows, inter, dtype=BF16, device="cuda")
    hip.op_gemm(abi.EPI_GEGLU_BF16, dev(x, BF16), dev(hip.interleave_geglu(wi), BF16), out)
    d = np.abs(host(out) - expect)
    assert np.all(d <= 4e-3 * np.abs(expect) + 2e-6), d.max()
    # and the oracle's fused GEGLU on the same values
    assert np.all(np.abs(oracle.linear_geglu(x, wi) - expect) <= 1e-5 * (1 + np.abs(expect)))


@pytest.mark.parametrize("n,k,epi", [(2304, 768, abi.EPI_STORE_BF16), (768, 768, abi.EPI_RESID_F32),
                                     (2304, 768, abi.EPI_GEGLU_BF16), (768, 1152, abi.EPI_RESID_F32)])
def test_gemm_sweep_shapes_full_size(n, k, epi):
    """The GEMM sweep's four shapes (configs[2]: Wqkv, attention-out + residual, Wi + GEGLU, MLP-out +
    residual) at M = 16384, where the persistent kernel walks several tiles per workgroup, against a torch
    FP32 product of the same bf16 operands on the GPU (FP32 accumulation order may differ; the bf16 outputs
    round once)."""
    M = 16384
    g = torch.Generator(device="cuda").manual_seed(n + k + epi)
    x = torch.randn(M, k, device="cuda", generator=g).to(BF16)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(BF16)
    prod = x.float() @ w.float().T
    if epi == abi.EPI_RESID_F32:
        base = torch.randn(M, n, device="cuda", generator=g)
        out = base.clone()
        hip.op_gemm(epi, x, w, out)
        torch.cuda.synchronize()
        assert (out - (base + prod)).abs().max().item() < 1e-4
        return
    if epi == abi.EPI_GEGLU_BF16:
        inter = n // 2
        expect = torch.nn.functional.gelu(prod[:, :inter]) * prod[:, inter:]
        wk = dev(hip.interleave_geglu(w.float().cpu().numpy()), BF16)
    else:
        expect, wk = prod, w
    out = torch.zeros(M, expect.shape[1], dtype=BF16, device="cuda")
    hip.op_gemm(epi, x, wk, out)
    torch.cuda.synchronize()
    d = (out.float() - expect).abs()
    assert bool((d <= 4e-3 * expect.abs() + 1e-5).all()), d.max().item()


def _check_wide_gemm(rows, n, k, epi, seed):
    """One GEMM of random bf16 operands through the C-ABI against a torch FP32 product of the same operands on the
    GPU, with the epilogue applied in FP32 (bf16 outputs within 4e-3 relative, FP32 residual within 1e-4)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, k, device="cuda", generator=g).to(BF16)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(BF16)
    prod = x.float() @ w.float().T
    if epi == abi.EPI_RESID_F32:
        base = torch.randn(rows, n, device="cuda", generator=g)
        out = base.clone()
        hip.op_gemm(epi, x, w, out)
        torch.cuda.synchronize()
        assert (out - (base + prod)).abs().max().item() < 1e-4
        return
    if epi == abi.EPI_BIAS_F32:
        bias = torch.randn(n, device="cuda", generator=g) * 0.1
        out = torch.full((rows, n), float("nan"), device="cuda")
        hip.op_gemm(epi, x, w, out, bias=bias)
        torch.cuda.synchronize()
        assert (out - (prod + bias)).abs().max().item() < 1e-4
        return
    kw, wk, scale = {}, w, None
    if epi == abi.EPI_GEGLU_BF16:
        inter = n // 2
        expect = torch.nn.functional.gelu(prod[:, :inter]) * prod[:, inter:]
        wk = dev(hip.interleave_geglu(w.float().cpu().numpy()), BF16)
    elif epi in (abi.EPI_BIAS_BF16, abi.EPI_BIAS_RELU_BF16):
        bias = torch.randn(n, device="cuda", generator=g) * 0.1
        expect = prod + bias
        if epi == abi.EPI_BIAS_RELU_BF16:
            expect = expect.clamp_min(0.0)
        kw = dict(bias=bias)
    elif epi == abi.EPI_ROPE_BF16:
        rc = 2 * n // 3  # q and k rotated, v not
        pos = torch.randint(0, 512, (rows,), device="cuda", generator=g, dtype=torch.int32)
        cos, sin = (dev(t) for t in oracle.rope_table(10000.0, 8192))
        expect = prod.clone()
        c, sn = cos[pos.long()], sin[pos.long()]
        scale = prod.abs().clone()
        for hd in range(0, rc, 64):
            a, b = prod[:, hd:hd + 32], prod[:, hd + 32:hd + 64]
            expect[:, hd:hd + 32] = a * c - b * sn
            expect[:, hd + 32:hd + 64] = b * c + a * sn
            m = a.abs() + b.abs()
            scale[:, hd:hd + 32] = m
            scale[:, hd + 32:hd + 64] = m
        kw = dict(pos=pos, cos=cos, sin=sin, rope_cols=rc)
    else:
        expect = prod
    out = torch.zeros(rows, expect.shape[1], dtype=BF16, device="cuda")
    hip.op_gemm(epi, x, wk, out, **kw)
    torch.cuda.synchronize()
    d = (out.float() - expect).abs()
    ref = scale if scale is not None else expect.abs()
    assert bool((d <= 4e-3 * ref + 1e-5).all()), d.max().item()


@pytest.mark.parametrize("rows,n,k,epi", [(24000, 768, 768, abi.EPI_STORE_BF16), (24000, 768, 768, abi.EPI_ROPE_BF16),
                                          (24000, 768, 768, abi.EPI_GEGLU_BF16), (24000, 768, 768, abi.EPI_BIAS_BF16),
                                          (24000, 768, 768, abi.EPI_RESID_F32)])
def test_gemm_192_token_tiles(rows, n, k, epi):
    """Shapes whose persistent GEMM runs 128-feature x 192-token tiles (24000 x 768: 750 tiles, 2 rounds of the
    512 resident workgroups against 3 for 128x128 tiles; N < 1024 never takes the eight-wave kernel), every
    epilogue family, against torch FP32."""
    _check_wide_gemm(rows, n, k, epi, rows + n + epi)


@pytest.mark.parametrize("rows,n,k,epi", [(9482, 2304, 768, abi.EPI_STORE_BF16), (9482, 2304, 768, abi.EPI_GEGLU_BF16),
                                          (9482, 2304, 768, abi.EPI_ROPE_BF16), (9482, 2304, 768, abi.EPI_BIAS_BF16),
                                          (7556, 1152, 384, abi.EPI_ROPE_BF16), (7556, 2304, 384, abi.EPI_GEGLU_BF16),
                                          (16500, 1152, 384, abi.EPI_BIAS_RELU_BF16),
                                          (32768, 2304, 768, abi.EPI_STORE_BF16), (32768, 2304, 768, abi.EPI_GEGLU_BF16),
                                          (23000, 1536, 128, abi.EPI_ROPE_BF16), (15000, 1152, 64, abi.EPI_ROPE_BF16),
                                          (30000, 2304, 64, abi.EPI_GEGLU_BF16),
                                          (12000, 2304, 768, abi.EPI_STORE_BF16), (11000, 1536, 768, abi.EPI_ROPE_BF16),
                                          (24000, 1152, 256, abi.EPI_GEGLU_BF16),
                                          (9482, 2304, 768, abi.EPI_RESID_F32), (12000, 1152, 768, abi.EPI_BIAS_F32)])
def test_gemm_eight_wave_tiles(rows, n, k, epi):
    """Shapes routed to the eight-wave 256-feature GEMM: 256x192 tiles at config1's 9482 tokens, at the Julia-1
    widths (N = 1152 leaves half a 256-feature tile, whose rows past N read as zeros from the buffer range check)
    and with token tiles cut at the end, and 256x256 tiles at 32768 tokens; every epilogue family, the FP32 ones
    (residual add, bias) at widths that reach this kernel (N = 768 stays on the four-wave kernels), against torch
    FP32.  The 23000 / 15000 / 30000 shapes run
    one or two K steps per tile with two to four tiles per workgroup, so the next tile's first stage is issued in
    the tile's first step and the RoPE position/cos/sin prefetch runs in the step that also waits on the previous
    epilogue.  Two-phase schedules (a round of full-height tiles, then a round of tiles 32 tokens shorter, whose
    loader waves multiply one 32-token block fewer): 192/160 at 9482 x 2304, 16500 x 1152, 15000 x 1152 (one K
    step) and 11000 x 1536; 256/224 at 12000 x 2304 and 24000 x 1152."""
    _check_wide_gemm(rows, n, k, epi, rows + 3 * n + epi)


@pytest.mark.parametrize("theta", [10000.0, 160000.0])
def test_gemm_rope(theta):
    r = rng(6)
    rows, h, k = 150, 256, 256
    n = 3 * h
    x, w, ref = _gemm_inputs(r, rows, n, k)
    pos = r.integers(0, 8192, rows).astype(np.int32)
    cos, sin = oracle.rope_table(theta, 8192)
    expect = ref.copy()
    for hd in range(0, 2 * h, 64):
        a, b = ref[:, hd:hd + 32], ref[:, hd + 32:hd + 64]
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        expect[:, hd:hd + 32] = a * c - b * s
        expect[:, hd + 32:hd + 64] = b * c + a * s
    scale = np.abs(ref).copy()
    for hd in range(0, 2 * h, 64):
        m = np.abs(ref[:, hd:hd + 32]) + np.abs(ref[:, hd + 32:hd + 64])
        scale[:, hd:hd + 32] = m
        scale[:, hd + 32:hd + 64] = m
    out = torch.zeros(rows, n, dtype=BF16, device="cuda")
    hip.op_gemm(abi.EPI_ROPE_BF16, dev(x, BF16), dev(w, BF16), out, pos=dev(pos), cos=dev(cos), sin=dev(sin),
                rope_cols=2 * h)
    d = np.abs(host(out) - expect)
    assert np.all(d <= 4e-3 * scale + 1e-6), d.max()


@pytest.mark.parametrize("splits,k,rows", [(0, 1152, 70), (2, 1152, 70), (5, 1152, 70),
                                           (0, 768, 70), (0, 384, 1), (0, 384, 33), (0, 512, 70), (0, 128, 5)])
@pytest.mark.parametrize("epi", [abi.EPI_STORE_BF16, abi.EPI_ROPE_BF16, abi.EPI_GEGLU_BF16, abi.EPI_RESID_F32,
                                 abi.EPI_BIAS_BF16, abi.EPI_BIAS_RELU_BF16, abi.EPI_BIAS_F32])
def test_gemm_splitk_matches_f64(epi, splits, k, rows):
    """Small-batch GEMMs against the f64 product, with the same per-epilogue tolerances as the single-pass
    GEMM, plus determinism: split-K (FP32 partials reduced in chunk order, then the epilogue) for a forced
    split count and for the paired epilogues at K = 1152, and the one-launch small-batch kernel (K split
    over the four waves of a workgroup, reduced in wave order) with the split count left to the library:
    32-feature tiles up to K = 1152 for the unpaired epilogues, 64-feature tiles up to K = 768."""
    r = rng(12)
    n = 384
    x, w, ref = _gemm_inputs(r, rows, n, k)
    bias = (r.standard_normal(n, dtype=np.float32) * 0.1).astype(np.float32)
    pos = r.integers(0, 8192, rows).astype(np.int32)
    cos, sin = oracle.rope_table(10000.0, 8192)
    ws = torch.zeros(8 << 20, dtype=torch.uint8, device="cuda")
    kw = {}
    if epi == abi.EPI_ROPE_BF16:
        kw = dict(pos=dev(pos), cos=dev(cos), sin=dev(sin), rope_cols=256)
        expect = ref.copy()
        scale = np.abs(ref).copy()
        for hd in range(0, 256, 64):
            a, b = ref[:, hd:hd + 32], ref[:, hd + 32:hd + 64]
            c, s_ = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
            expect[:, hd:hd + 32] = a * c - b * s_
            expect[:, hd + 32:hd + 64] = b * c + a * s_
            scale[:, hd:hd + 64] = np.tile(np.abs(a) + np.abs(b), 2)
    elif epi == abi.EPI_GEGLU_BF16:
        wi = w
        prod = x.astype(np.float64) @ wi.astype(np.float64).T
        u, v = prod[:, :n // 2], prod[:, n // 2:]
        erf = np.vectorize(math.erf)
        expect = 0.5 * u * (1 + erf(u / math.sqrt(2))) * v
        scale = np.abs(expect) + 1e-3 * np.abs(u * v)
        w = hip.interleave_geglu(wi)
    elif epi == abi.EPI_RESID_F32:
        base = r.standard_normal((rows, n), dtype=np.float32)
        kw = dict(bias=dev(bias))
        expect = base + ref + bias
    else:
        kw = dict(bias=dev(bias)) if epi != abi.EPI_STORE_BF16 else {}
        expect = ref + (bias if kw else 0)
        if epi == abi.EPI_BIAS_RELU_BF16:
            expect = np.maximum(expect, 0)
    width = n // 2 if epi == abi.EPI_GEGLU_BF16 else n
    f32 = epi in (abi.EPI_RESID_F32, abi.EPI_BIAS_F32)
    outs = []
    for _ in range(2):
        out = dev(base) if epi == abi.EPI_RESID_F32 else torch.zeros(rows, width, dtype=torch.float32 if f32 else BF16,
                                                                      device="cuda")
        hip.op_gemm_splitk(epi, dev(x, BF16), dev(w, BF16), out, ws, splits=splits, **kw)
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])  # fixed reduction order
    d = np.abs(outs[0] - expect)
    if f32:
        assert d.max() < 1e-4, d.max()
    else:
        sc = scale if epi in (abi.EPI_ROPE_BF16, abi.EPI_GEGLU_BF16) else np.abs(expect)
        assert np.all(d <= 4e-3 * sc + 2e-6), d.max()


@pytest.mark.parametrize("splits", [4, 0])
def test_gemm_splitk_gathered_rows(splits):
    """Row-gathered X through the split-K pass (splits=4) and through the one-launch small-batch kernel."""
    r = rng(13)
    x, w, ref = _gemm_inputs(r, 300, 256, 512)
    idx = np.array([5, 0, 299, 17, 17, 100, 3], dtype=np.int32)
    out = torch.zeros(idx.size, 256, dtype=torch.float32, device="cuda")
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    hip.op_gemm_splitk(abi.EPI_BIAS_F32, dev(x, BF16), dev(w, BF16), out, ws, splits=splits, rows=idx.size,
                       gather=dev(idx), bias=dev(np.zeros(256, dtype=np.float32)))
    assert np.abs(host(out) - ref[idx]).max() < 1e-5


@pytest.mark.parametrize("rows,n,epi", [(300, 2304, abi.EPI_STORE_BF16), (300, 2304, abi.EPI_RESID_F32),
                                        (300, 2304, abi.EPI_BIAS_F32), (130, 8192, abi.EPI_BIAS_RELU_BF16)])
def test_gemm_small_wide_outputs(rows, n, epi):
    """The one-launch small-batch kernel on 64-feature tiles for epilogues without a feature pairing (taken
    when 32-feature tiles would not fit one workgroup per CU), against torch FP32."""
    _check_small(rows, n, 768, epi, seed=rows + n + epi)


def _check_small(rows, n, k, epi, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    x = torch.randn(rows, k, device="cuda", generator=g).to(BF16)
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(BF16)
    bias = torch.randn(n, device="cuda", generator=g) * 0.1
    prod = x.float() @ w.float().T + (bias if epi != abi.EPI_STORE_BF16 else 0)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    kw = dict(bias=bias) if epi != abi.EPI_STORE_BF16 else {}
    if epi == abi.EPI_RESID_F32:
        base = torch.randn(rows, n, device="cuda", generator=g)
        out = base.clone()
        hip.op_gemm_splitk(epi, x, w, out, ws, **kw)
        torch.cuda.synchronize()
        assert (out - (base + prod)).abs().max().item() < 1e-4
        return
    f32 = epi == abi.EPI_BIAS_F32
    out = torch.zeros(rows, n, dtype=torch.float32 if f32 else BF16, device="cuda")
    hip.op_gemm_splitk(epi, x, w, out, ws, **kw)
    expect = prod.clamp_min(0.0) if epi == abi.EPI_BIAS_RELU_BF16 else prod
    d = (out.float() - expect).abs()
    if f32:
        assert d.max().item() < 1e-4
    else:
        assert bool((d <= 4e-3 * expect.abs() + 1e-5).all()), d.max().item()


@pytest.mark.parametrize("rows,hidden,n,epi,biased,pad", [
    (128, 768, 2304, abi.EPI_ROPE_BF16, False, 0), (128, 768, 2304, abi.EPI_GEGLU_BF16, False, 0),
    (160, 384, 1152, abi.EPI_ROPE_BF16, False, 0), (160, 384, 2304, abi.EPI_GEGLU_BF16, False, 0),
    (1, 128, 384, abi.EPI_ROPE_BF16, True, 4), (33, 256, 512, abi.EPI_GEGLU_BF16, True, 0),
    (70, 512, 1536, abi.EPI_ROPE_BF16, False, 8), (230, 768, 1152, abi.EPI_STORE_BF16, True, 0)])
def test_gemm_layer_norm_prologue(rows, hidden, n, epi, biased, pad):
    """The LayerNorm prologue of the small-batch GEMM gives the same bits as jh_op_layer_norm followed by the
    same GEMM (bf16 operand, same K-slice order), for the hidden sizes it supports, LayerNorm with and without
    bias, rows not a multiple of 32 and a row stride past K; plus torch FP32 of the same bf16 operand."""
    g = torch.Generator(device="cuda").manual_seed(rows + hidden + n + epi)
    xf_full = torch.randn(rows, hidden + pad, device="cuda", generator=g) * 3.0 + 0.5
    xf = xf_full[:, :hidden]
    ln_w = torch.rand(hidden, device="cuda", generator=g) + 0.5
    ln_b = torch.randn(hidden, device="cuda", generator=g) * 0.1 if biased else None
    w = (torch.randn(n, hidden, device="cuda", generator=g) * 0.02).to(BF16)
    wk = dev(hip.interleave_geglu(w.float().cpu().numpy()), BF16) if epi == abi.EPI_GEGLU_BF16 else w
    xn = torch.zeros(rows, hidden, dtype=BF16, device="cuda")
    hip.op_layer_norm(xf.contiguous(), ln_w, ln_b, 1e-5, xn)
    kw = {}
    if epi == abi.EPI_ROPE_BF16:
        pos = torch.randint(0, 8192, (rows,), device="cuda", generator=g, dtype=torch.int32)
        cos, sin = (dev(t) for t in oracle.rope_table(160000.0, 8192))
        kw = dict(pos=pos, cos=cos, sin=sin, rope_cols=2 * n // 3)
    width = n // 2 if epi == abi.EPI_GEGLU_BF16 else n
    got = torch.zeros(rows, width, dtype=BF16, device="cuda")
    hip.op_gemm_ln(epi, xf_full, wk, got, ln_w, ln_b, 1e-5, rows=rows, **kw)
    ref = torch.zeros_like(got)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    hip.op_gemm_splitk(epi, xn, wk, ref, ws, **kw)
    torch.cuda.synchronize()
    if epi != abi.EPI_STORE_BF16:  # same kernel family and tile: identical
        assert torch.equal(got, ref)
    prod = xn.float() @ w.float().T
    if epi == abi.EPI_GEGLU_BF16:
        expect = torch.nn.functional.gelu(prod[:, :n // 2]) * prod[:, n // 2:]
        scale = expect.abs() + 1e-3 * (prod[:, :n // 2] * prod[:, n // 2:]).abs()
    elif epi == abi.EPI_ROPE_BF16:
        rc = 2 * n // 3
        expect, scale = prod.clone(), prod.abs().clone()
        c, sn = kw["cos"][kw["pos"].long()], kw["sin"][kw["pos"].long()]
        for hd in range(0, rc, 64):
            a, b = prod[:, hd:hd + 32], prod[:, hd + 32:hd + 64]
            expect[:, hd:hd + 32] = a * c - b * sn
            expect[:, hd + 32:hd + 64] = b * c + a * sn
            scale[:, hd:hd + 64] = (a.abs() + b.abs()).repeat(1, 2)
    else:
        expect, scale = prod, prod.abs()
    d = (got.float() - expect).abs()
    assert bool((d <= 4e-3 * scale + 1e-5).all()), d.max().item()


def test_gemm_layer_norm_prologue_rejects():
    xf = torch.zeros(4, 192, device="cuda")
    w = torch.zeros(128, 192, dtype=BF16, device="cuda")
    out = torch.zeros(4, 128, dtype=BF16, device="cuda")
    ln_w = torch.ones(192, device="cuda")
    with pytest.raises(hip.HipError):  # hidden 192 has no prologue instance
        hip.op_gemm_ln(abi.EPI_STORE_BF16, xf, w, out, ln_w)
    xf = torch.zeros(4, 128, device="cuda")
    w = torch.zeros(128, 128, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):  # residual epilogue: not a prologue epilogue
        hip.op_gemm_ln(abi.EPI_RESID_F32, xf, w, torch.zeros(4, 128, device="cuda"), ln_w[:128])
    with pytest.raises(hip.HipError):  # no LayerNorm weights
        hip.op_gemm_ln(abi.EPI_STORE_BF16, xf, w, out, None)


def test_gemm_rejects_bad_shapes():
    x = torch.zeros(4, 100, dtype=BF16, device="cuda")
    w = torch.zeros(64, 100, dtype=BF16, device="cuda")
    out = torch.zeros(4, 64, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):
        hip.op_gemm(abi.EPI_STORE_BF16, x, w, out)
    # output column not on a 16-byte boundary
    x = torch.zeros(4, 64, dtype=BF16, device="cuda")
    out = torch.zeros(4, 72, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):
        hip.op_gemm(abi.EPI_STORE_BF16, x, w, out, col=4)


@pytest.mark.parametrize("hidden", [128, 384, 768])
def test_embed_and_layer_norm(hidden):
    r = rng(7)
    vocab, rows = 1000, 333
    table = r.standard_normal((vocab, hidden), dtype=np.float32) * 0.02
    w = 1 + 0.1 * r.standard_normal(hidden, dtype=np.float32)
    b = 0.1 * r.standard_normal(hidden, dtype=np.float32)
    ids = r.integers(0, vocab, rows).astype(np.uint32)
    x = torch.zeros(rows, hidden, device="cuda")
    xn = torch.zeros(rows, hidden, dtype=BF16, device="cuda")
    hip.op_embed_ln(dev(ids.astype(np.int32)), dev(table), dev(w), 1e-5, x, xn)
    expect = oracle.layer_norm(table[ids], w, None, 1e-5)
    assert np.abs(host(x) - expect).max() < 2e-5
    assert np.all(np.abs(host(xn) - expect) <= 4e-3 * np.abs(expect) + 1e-6)
    # f64 closed form
    t = table[ids].astype(np.float64)
    ln = (t - t.mean(1, keepdims=True)) / np.sqrt(t.var(1, keepdims=True) + 1e-5) * w
    assert np.abs(host(x) - ln).max() < 2e-5
    out = torch.zeros(rows, hidden, dtype=BF16, device="cuda")
    xs = r.standard_normal((rows, hidden), dtype=np.float32) * 3 + 1
    hip.op_layer_norm(dev(xs), dev(w), dev(b), 1e-5, out)
    expect = oracle.layer_norm(xs, w, b, 1e-5)
    assert np.all(np.abs(host(out) - expect) <= 4e-3 * np.abs(expect) + 1e-5)


@pytest.mark.parametrize("rows", [1, 3, 5, 29, 32, 33, 64, 71, 4096, 4099])
def test_layer_norm_covers_every_row(rows):
    """The LayerNorm kernel deals its 8-row workgroups (two rows per wave) to the XCDs in contiguous eighths
    (workgroup b on XCD b % 8); every row must still be written exactly as the oracle's LayerNorm, for grids of
    fewer than 8 workgroups, exactly 8 and 512 workgroups, a partial last workgroup, and a wave whose second row
    is past the end (output pre-filled with NaN so a skipped row shows)."""
    r = rng(100 + rows)
    hidden = 768
    xs = r.standard_normal((rows, hidden), dtype=np.float32) * 2 + 0.5
    w = 1 + 0.1 * r.standard_normal(hidden, dtype=np.float32)
    b = 0.1 * r.standard_normal(hidden, dtype=np.float32)
    out = torch.full((rows, hidden), float("nan"), dtype=BF16, device="cuda")
    hip.op_layer_norm(dev(xs), dev(w), dev(b), 1e-5, out)
    got = host(out)
    expect = oracle.layer_norm(xs, w, b, 1e-5)
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - expect) <= 4e-3 * np.abs(expect) + 1e-5)


def test_final_norm_and_scorer():
    r = rng(8)
    rows, hidden = 97, 768
    x0 = r.standard_normal((rows, hidden), dtype=np.float32)
    fw = 1 + 0.1 * r.standard_normal(hidden, dtype=np.float32)
    te = 0.02 * r.standard_normal((3, hidden), dtype=np.float32)
    hw = 1 + 0.1 * r.standard_normal(hidden, dtype=np.float32)
    hb = 0.1 * r.standard_normal(hidden, dtype=np.float32)
    qt = r.integers(0, 3, rows)
    pos = r.integers(0, 8192, rows)
    meta = (pos | (qt << 16)).astype(np.uint32)
    x = dev(x0)
    out = torch.zeros(rows, hidden, dtype=BF16, device="cuda")
    hip.op_final_norm(x, dev(fw), dev(te), dev(meta.astype(np.int32)), dev(hw), dev(hb), 1e-5, out)
    x1 = oracle.layer_norm(x0, fw, None, 1e-5) + te[qt]
    assert np.abs(host(x) - x1).max() < 2e-5
    e2 = oracle.layer_norm(x1, hw, hb, 1e-5)
    assert np.all(np.abs(host(out) - e2) <= 4e-3 * np.abs(e2) + 1e-5)
    # gather + scorer
    idx = np.array([3, 1, 96, 50], dtype=np.int32)
    dst = torch.zeros(idx.size, hidden, device="cuda")
    hip.op_gather_f32(x, dev(idx), dst)
    assert np.array_equal(host(dst), host(x)[idx])
    z = r.standard_normal((rows, hidden), dtype=np.float32)
    w2 = 0.02 * r.standard_normal(hidden, dtype=np.float32)
    s = torch.zeros(rows, device="cuda")
    hip.op_scorer(dev(z), dev(w2), 0.25, s)
    erf = np.vectorize(math.erf)
    z64 = z.astype(np.float64)
    expect = (0.5 * z64 * (1 + erf(z64 / math.sqrt(2))) * w2).sum(1) + 0.25
    assert np.abs(host(s) - expect).max() < 1e-4


def _attn_ref64(q, k, v, seqs, heads, window, scale=0.125):
    """f64 softmax(scale·QKᵀ + mask)·V per (sequence, head); seqs = (q_row, nq, kv_row, len, q_pos)."""
    out = np.zeros((q.shape[0], heads * 64))
    for q_row, nq, kv_row, ln, q_pos in seqs:
        for hh in range(heads):
            Q = q[q_row:q_row + nq, hh * 64:(hh + 1) * 64].astype(np.float64)
            K = k[kv_row:kv_row + ln, hh * 64:(hh + 1) * 64].astype(np.float64)
            V = v[kv_row:kv_row + ln, hh * 64:(hh + 1) * 64].astype(np.float64)
            s = scale * Q @ K.T
            if window >= 0:
                qp = q_pos + np.arange(nq)[:, None]
                kp = np.arange(ln)[None, :]
                s = np.where(np.abs(qp - kp) <= window, s, -np.inf)
            s = s - s.max(1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(1, keepdims=True)
            out[q_row:q_row + nq, hh * 64:(hh + 1) * 64] = p @ V
    return out


def _tiles(lens, qt=64):
    tiles, start = [], 0
    for ln in lens:
        for q0 in range(0, ln, qt):
            tiles.append((start + q0, min(qt, ln - q0), start, ln, q0))
        start += ln
    return tiles


@pytest.mark.parametrize("qt", [64, 128])
@pytest.mark.parametrize("window", [-1, 64, 8, 0])
def test_attention_varlen(window, qt):
    r = rng(9)
    heads = 3
    h = heads * 64
    lens = [1, 5, 63, 64, 65, 127, 128, 129, 200, 300]
    t = sum(lens)
    qkv = bf16_round(r.standard_normal((t, 3 * h), dtype=np.float32))
    q, k, v = qkv[:, :h], qkv[:, h:2 * h], qkv[:, 2 * h:]
    tiles = _tiles(lens, qt)
    seqs = []
    start = 0
    for ln in lens:
        seqs.append((start, ln, start, ln, 0))
        start += ln
    expect = _attn_ref64(q, k, v, seqs, heads, window)
    dq = dev(qkv, BF16)
    out = torch.zeros(t, h, dtype=BF16, device="cuda")
    hip.op_attention(dq, 3 * h, dq[:, h:], dq[:, 2 * h:], 3 * h, out, h, dev(np.array(tiles, dtype=np.int32)), heads,
                     window)
    got = host(out)
    assert np.abs(got - expect).max() < 2e-2, np.abs(got - expect).max()
    # the oracle's attention on the same values, same window semantics
    orc = oracle.attention(qkv, qkv, [(s[0], s[1], s[2], s[3]) for s in seqs], heads, window)
    assert np.abs(orc - expect).max() < 1e-4


@pytest.mark.parametrize("window", [-1, 64])
def test_attention_wide_items(window):
    """jh_op_attention_wide (eight waves, up to 256 queries per work item; the backend's global layers of long
    sequences) on ragged lengths: each query's keys are visited in the same 64-key tiles as with 128-query items,
    so the output equals jh_op_attention's bit for bit, and both are within 2e-2 of the f64 reference."""
    r = rng(31)
    heads = 2
    h = heads * 64
    lens = [1, 100, 129, 255, 256, 257, 511, 700, 1300]
    t = sum(lens)
    qkv = bf16_round(r.standard_normal((t, 3 * h), dtype=np.float32))
    seqs, start = [], 0
    for ln in lens:
        seqs.append((start, ln, start, ln, 0))
        start += ln
    expect = _attn_ref64(qkv[:, :h], qkv[:, h:2 * h], qkv[:, 2 * h:], seqs, heads, window)
    dq = dev(qkv, BF16)
    outs = []
    for qt, wide in ((128, False), (256, True)):
        out = torch.zeros(t, h, dtype=BF16, device="cuda")
        hip.op_attention(dq, 3 * h, dq[:, h:], dq[:, 2 * h:], 3 * h, out, h,
                         dev(np.array(_tiles(lens, qt), dtype=np.int32)), heads, window, wide=wide)
        outs.append(host(out))
    assert np.array_equal(outs[0], outs[1])
    assert np.abs(outs[1] - expect).max() < 2e-2, np.abs(outs[1] - expect).max()


@pytest.mark.parametrize("window", [-1, 64])
def test_attention_rising_scores(window):
    """Scores that climb along each sequence at several rates (about 2 to 40 log2 units per 64-key tile), so the
    running max must move again and again after the first tile: every rescale case of the online softmax (a rise
    within the lazy threshold, just past it, far past it, to where exp2 would overflow without one) against f64."""
    r = rng(11)
    heads = 2
    h = heads * 64
    lens = [300, 257, 300, 190, 300]
    rates = [0.15, 0.5, 0.8, 1.3, 3.0]  # beta rise per 64 keys
    t = sum(lens)
    q = np.abs(r.standard_normal((t, h))) + 0.5
    u = np.abs(r.standard_normal(h)) + 0.5
    k = 0.3 * r.standard_normal((t, h))
    start = 0
    for ln, rate in zip(lens, rates):
        beta = rate * np.arange(ln) / 64.0
        k[start:start + ln] += beta[:, None] * u[None, :]
        start += ln
    v = r.standard_normal((t, h))
    qkv = bf16_round(np.concatenate([q, k, v], 1).astype(np.float32))
    q, k, v = qkv[:, :h], qkv[:, h:2 * h], qkv[:, 2 * h:]
    tiles = _tiles(lens, 128)
    seqs, start = [], 0
    for ln in lens:
        seqs.append((start, ln, start, ln, 0))
        start += ln
    expect = _attn_ref64(q, k, v, seqs, heads, window)
    dq = dev(qkv, BF16)
    out = torch.zeros(t, h, dtype=BF16, device="cuda")
    hip.op_attention(dq, 3 * h, dq[:, h:], dq[:, 2 * h:], 3 * h, out, h, dev(np.array(tiles, dtype=np.int32)), heads,
                     window)
    got = host(out)
    assert np.isfinite(got).all()
    assert np.abs(got - expect).max() < 2e-2, np.abs(got - expect).max()


@pytest.mark.parametrize("window", [-1, 512])
def test_attention_scores_far_above_running_max(window):
    """Single keys whose scores sit 12 to 15 log2 units above the running max (scores ~0 before them).  The fast
    path keeps a tile without computing its max while each lane's 32 values of p sum to at most 2^16, so it
    carries one p of up to 2^15 (keys 70 and 100 share a lane: 2^12 + 2^13.5); two keys at 15.5 units in one
    lane's 32 (keys 192, 193) exceed the bound and send that tile to the slow path, which moves the max; a spike in a
    sequence's last, partial tile (key 199 of 200) is masked on the slow path.  Against f64 softmax.  (Window 512
    covers both sequences, so no tile is a window edge and the fast path runs as for global attention.)"""
    r = rng(12)
    heads = 2
    h = heads * 64
    lens = [256, 200]
    t = sum(lens)
    c = 0.125 * math.log2(math.e)
    u = np.abs(r.standard_normal(h)) + 0.5
    q = u[None, :] + 0.05 * r.standard_normal((t, h))
    k = 0.05 * r.standard_normal((t, h))
    spikes = [(70, 12.0), (100, 13.5), (150, 15.0), (192, 15.5), (193, 15.5),
              (256 + 64, 14.0), (256 + 130, 12.5), (256 + 199, 15.0)]
    for row, d in spikes:
        for hh in range(heads):
            uh = u[hh * 64:(hh + 1) * 64]
            k[row, hh * 64:(hh + 1) * 64] = (d / c) * uh / (uh @ uh)
    v = r.standard_normal((t, h))
    qkv = bf16_round(np.concatenate([q, k, v], 1).astype(np.float32))
    q, k, v = qkv[:, :h], qkv[:, h:2 * h], qkv[:, 2 * h:]
    # the spikes stand where intended for every query and head (within 0.3 log2 units: the two at 15.5 still sum
    # past 2^16, a single one at 15 stays below it), the other keys below 1
    rows = [row for row, _ in spikes]
    for hh in range(heads):
        qh, kh = q[:, hh * 64:(hh + 1) * 64].astype(np.float64), k[:, hh * 64:(hh + 1) * 64].astype(np.float64)
        assert np.abs(c * qh @ kh[rows].T - [d for _, d in spikes]).max() < 0.3
        assert (c * qh @ np.delete(kh, rows, 0).T).max() < 1.0
    tiles = _tiles(lens, 128)
    seqs, start = [], 0
    for ln in lens:
        seqs.append((start, ln, start, ln, 0))
        start += ln
    expect = _attn_ref64(q, k, v, seqs, heads, window)
    dq = dev(qkv, BF16)
    out = torch.zeros(t, h, dtype=BF16, device="cuda")
    hip.op_attention(dq, 3 * h, dq[:, h:], dq[:, 2 * h:], 3 * h, out, h, dev(np.array(tiles, dtype=np.int32)), heads,
                     window)
    got = host(out)
    assert np.isfinite(got).all()
    assert np.abs(got - expect).max() < 2e-2, np.abs(got - expect).max()


@pytest.mark.parametrize("window", [-1, 64])
def test_attention_full_length_8192(window):
    """One 8192-token sequence with the ModernBERT-base heads, global and sliding-window, in the
    backend's 128-query tiles, against softmax(0.125·QKᵀ + mask)·V in FP32 on the GPU, head by head."""
    L, heads = 8192, 12
    h = heads * 64
    g = torch.Generator(device="cuda").manual_seed(8192 + window)
    qkv = torch.randn(L, 3 * h, device="cuda", generator=g).to(BF16)
    tiles = dev(np.array(_tiles([L], 128), dtype=np.int32))
    out = torch.zeros(L, h, dtype=BF16, device="cuda")
    hip.op_attention(qkv, 3 * h, qkv[:, h:], qkv[:, 2 * h:], 3 * h, out, h, tiles, heads, window)
    pos = torch.arange(L, device="cuda")
    worst = 0.0
    for hh in range(heads):
        q = qkv[:, hh * 64:(hh + 1) * 64].float()
        k = qkv[:, h + hh * 64:h + (hh + 1) * 64].float()
        v = qkv[:, 2 * h + hh * 64:2 * h + (hh + 1) * 64].float()
        s = 0.125 * (q @ k.T.contiguous())
        if window >= 0:
            s = s.masked_fill((pos[:, None] - pos[None, :]).abs() > window, float("-inf"))
        ref = torch.softmax(s, dim=1) @ v
        worst = max(worst, (out[:, hh * 64:(hh + 1) * 64].float() - ref).abs().max().item())
        del s, ref
    assert worst < 2e-2, worst


def test_attention_marker_queries():
    """Queries from a separate buffer (the marker-only head layer) against full keys."""
    r = rng(10)
    heads, h = 2, 128
    lens = [40, 130, 7]
    t = sum(lens)
    kv = bf16_round(r.standard_normal((t, 3 * h), dtype=np.float32))
    markers = [[1, 5, 39], list(range(0, 130, 2)), [0, 6]]
    nm = sum(len(m) for m in markers)
    qm = bf16_round(r.standard_normal((nm, h), dtype=np.float32))
    tiles, seqs, start, mi = [], [], 0, 0
    for ln, ms in zip(lens, markers):
        for j in range(0, len(ms), 64):
            tiles.append((mi + j, min(64, len(ms) - j), start, ln, 0))
        seqs.append((mi, len(ms), start, ln, 0))
        start += ln
        mi += len(ms)
    expect = _attn_ref64(qm, kv[:, h:2 * h], kv[:, 2 * h:], seqs, heads, -1)
    dkv = dev(kv, BF16)
    out = torch.zeros(nm, h, dtype=BF16, device="cuda")
    hip.op_attention(dev(qm, BF16), h, dkv[:, h:], dkv[:, 2 * h:], 3 * h, out, h,
                     dev(np.array(tiles, dtype=np.int32)), heads, -1)
    assert np.abs(host(out) - expect).max() < 2e-2
