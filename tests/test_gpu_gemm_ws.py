"""The weight-stationary GEMM (jh_op_gemm_ws, csrc/gemm_ws.hip) on the GPU.

Each case runs the same bf16 operands through jh_op_gemm_ws (W packed by
jh_op_pack_ws) and through jh_op_gemm (the tiled kernels), and requires:
- agreement between the two to FP32 summation order: both sum the same bf16
  products in K order (in MFMA steps of 32 and 16 products) and apply the same
  epilogue expressions, so bf16 outputs may differ by one rounding step
  (at most 2^-7 relative) and FP32 outputs by 1e-5;
- agreement with a torch FP32 product of the same operands on the GPU with the
  epilogue applied in FP32 (bf16 outputs within 4e-3 relative, FP32 residual
  outputs within 1e-4), so a mistake shared by both kernels is caught too.
Shapes cover config1's encoder GEMMs (9482 tokens), the M = 16384 sweep, and
token counts that leave one block per token range, a single workgroup per
slab, a partial last block, and ranges of unequal length.  At K = 1152 (the
MLP-out projection, residual epilogue only) the kernel splits K between
partner waves and adds the upper half's sums to the lower half's through LDS;
the same checks apply, and rows stay independent of the batch.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from julia1_amd import abi, hip  # noqa: E402
from oracle import oracle  # noqa: E402
from gpu_util import dev  # noqa: E402

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
K = 768


def _case(rows, n, epi, seed, bias=False, col=0, pad_out=0, ldx_pad=0, k=K):
    g = torch.Generator(device="cuda").manual_seed(seed)
    xs = torch.randn(rows, k + ldx_pad, device="cuda", generator=g).to(BF16)
    x = xs[:, :k]  # row stride k + ldx_pad
    w = (torch.randn(n, k, device="cuda", generator=g) * 0.02).to(BF16)
    prod = x.float() @ w.float().T
    kw = {}
    if epi == abi.EPI_GEGLU_BF16:
        inter = n // 2
        expect = torch.nn.functional.gelu(prod[:, :inter]) * prod[:, inter:]
        wk = dev(hip.interleave_geglu(w.float().cpu().numpy()), BF16)
        scale = expect.abs()
    else:
        wk = w
        expect, scale = prod.clone(), prod.abs().clone()
    if epi == abi.EPI_ROPE_BF16:
        rc = 2 * n // 3 // 64 * 64
        pos = torch.randint(0, 8192, (rows,), device="cuda", generator=g, dtype=torch.int32)
        cos, sin = (dev(t) for t in oracle.rope_table(10000.0, 8192))
        c, sn = cos[pos.long()], sin[pos.long()]
        for hd in range(0, rc, 64):
            a, b = prod[:, hd:hd + 32], prod[:, hd + 32:hd + 64]
            expect[:, hd:hd + 32] = a * c - b * sn
            expect[:, hd + 32:hd + 64] = b * c + a * sn
            m = a.abs() + b.abs()
            scale[:, hd:hd + 32] = m
            scale[:, hd + 32:hd + 64] = m
        kw = dict(pos=pos, cos=cos, sin=sin, rope_cols=rc)
    if bias or epi in (abi.EPI_BIAS_BF16, abi.EPI_BIAS_RELU_BF16, abi.EPI_BIAS_F32):
        b = torch.randn(n, device="cuda", generator=g) * 0.1
        kw["bias"] = b
        expect = expect + b
        scale = scale + b.abs()
        if epi == abi.EPI_BIAS_RELU_BF16:
            expect = expect.clamp_min(0.0)
    f32 = epi in (abi.EPI_RESID_F32, abi.EPI_BIAS_F32)
    width = expect.shape[1]
    if f32:
        base = torch.randn(rows, width + col + pad_out, device="cuda", generator=g)
        if epi == abi.EPI_BIAS_F32:
            base.zero_()
        out_ws, out_ref = base.clone(), base.clone()
        if epi == abi.EPI_RESID_F32:
            expect = expect + base[:, col:col + width]
    else:
        out_ws = torch.zeros(rows, width + col + pad_out, dtype=BF16, device="cuda")
        out_ref = out_ws.clone()
    wp = hip.pack_ws(wk)
    hip.op_gemm_ws(epi, x, wp, n, k, out_ws, col=col, **kw)
    hip.op_gemm(epi, x, wk, out_ref, col=col, **kw)
    torch.cuda.synchronize()
    dk = (out_ws.float() - out_ref.float()).abs()
    if f32:
        assert dk.max().item() <= 1e-5, dk.max().item()
    else:
        lim = torch.maximum(out_ws.float().abs(), out_ref.float().abs()) * 2.0 ** -7 + 1e-6  # one bf16 step
        assert bool((dk <= lim).all()), dk.max().item()
    got = out_ws[:, col:col + width].float()
    d = (got - expect).abs()
    if f32:
        assert d.max().item() < 1e-4
    else:
        assert bool((d <= 4e-3 * scale + 1e-5).all()), d.max().item()
    # columns outside [col, col + width) untouched
    if col:
        assert torch.equal(out_ws[:, :col], out_ref[:, :col])
    if pad_out:
        assert torch.equal(out_ws[:, col + width:], out_ref[:, col + width:])
    # deterministic: a second run gives the same bits
    again = out_ref.clone() if not f32 else base.clone()
    if not f32:
        again.zero_()
    hip.op_gemm_ws(epi, x, wp, n, k, again, col=col, **kw)
    torch.cuda.synchronize()
    assert torch.equal(again, out_ws)


@pytest.mark.parametrize("rows,n,epi", [(9482, 2304, abi.EPI_ROPE_BF16), (9482, 2304, abi.EPI_GEGLU_BF16),
                                        (9482, 768, abi.EPI_RESID_F32), (9482, 2304, abi.EPI_STORE_BF16),
                                        (9482, 2304, abi.EPI_BIAS_BF16), (9482, 3072, abi.EPI_BIAS_RELU_BF16),
                                        (9482, 768, abi.EPI_BIAS_F32), (9482, 1536, abi.EPI_BIAS_BF16)])
def test_ws_config1_shapes(rows, n, epi):
    """config1's encoder GEMMs (Wqkv + RoPE, Wi + GEGLU, Wo + residual) and the head's K = 768 projections."""
    _case(rows, n, epi, seed=rows + n + epi)


@pytest.mark.parametrize("epi", [abi.EPI_ROPE_BF16, abi.EPI_GEGLU_BF16, abi.EPI_RESID_F32])
def test_ws_sweep_size(epi):
    """M = 16384 (the GEMM sweep): 19 or 18 blocks per token range."""
    _case(16384, 2304 if epi != abi.EPI_RESID_F32 else 768, epi, seed=16384 + epi)


@pytest.mark.parametrize("rows", [1, 31, 33, 64, 100, 257, 1000, 2000, 8197])
@pytest.mark.parametrize("epi", [abi.EPI_ROPE_BF16, abi.EPI_GEGLU_BF16, abi.EPI_RESID_F32])
def test_ws_token_counts(rows, epi):
    """16-token blocks: a single block (1), one block per range (31 .. 257: 2 to 17 ranges per slab), ranges of
    2 or 3 blocks (1000), 4 or 5 (2000) and 18 or 19 (8197), so both the paired block loop and its odd tail run,
    and a partial last block (every count not a multiple of 16)."""
    _case(rows, 2304 if epi != abi.EPI_RESID_F32 else 768, epi, seed=rows * 7 + epi)


@pytest.mark.parametrize("epi", [abi.EPI_ROPE_BF16, abi.EPI_RESID_F32, abi.EPI_STORE_BF16])
def test_ws_strided_rows_and_column_offset(epi):
    """X with a row stride above K, the output written from a column offset with columns on either side."""
    _case(3001, 768, epi, seed=99 + epi, bias=epi == abi.EPI_RESID_F32, col=16, pad_out=8, ldx_pad=64)


def test_ws_rejects_unsupported_shapes():
    x = torch.zeros(64, 384, dtype=BF16, device="cuda")
    w = torch.zeros(256, 384, dtype=BF16, device="cuda")
    out = torch.zeros(64, 256, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):
        hip.op_gemm_ws(abi.EPI_STORE_BF16, x, w, 256, 384, out)  # K != 768
    x = torch.zeros(64, K, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):
        hip.op_gemm_ws(abi.EPI_STORE_BF16, x, torch.zeros(192, K, dtype=BF16, device="cuda"), 192, K, out)
    with pytest.raises(hip.HipError):
        hip.pack_ws(torch.zeros(192, K, dtype=BF16))


def test_pack_ws_layout():
    """The packed order on the host: slab f, wave w, slice s, half h, lane l holds W row
    64(4f + w/2) + 32h + 16(w % 2) + l % 16, K 32s + 8(l/16) .. +8."""
    n = 512
    w = torch.arange(n * K, dtype=torch.int32).remainder(65521).to(torch.int16).view(BF16).reshape(n, K)
    p = hip.pack_ws(w).cpu().view(torch.int16).numpy().reshape(n // 256, 8, K // 32, 2, 64, 8)
    src = w.view(torch.int16).numpy()
    rng = np.random.default_rng(5)
    for _ in range(300):
        f, wv, s = rng.integers(0, n // 256), rng.integers(0, 8), rng.integers(0, K // 32)
        h, ln = rng.integers(0, 2), rng.integers(0, 64)
        rw = 64 * (4 * f + wv // 2) + 32 * h + 16 * (wv % 2) + ln % 16
        k0 = 32 * s + 8 * (ln // 16)
        assert np.array_equal(p[f, wv, s, h, ln], src[rw, k0:k0 + 8])


@pytest.mark.parametrize("epi", [abi.EPI_ROPE_BF16, abi.EPI_GEGLU_BF16, abi.EPI_RESID_F32, abi.EPI_BIAS_BF16,
                                 abi.EPI_STORE_BF16])
def test_ws_rows_independent_of_batch(epi):
    """A token's outputs are the same bits whatever else is in the batch: rows of sub-batches (config1's first
    sequence lengths, at their offsets in a 2147-token batch, so a token sits at another place in its 16-token
    block and its block at another place in its token range) equal the same rows of the full batch.  The
    encoder's batching invariance (src tests/checkpoint.rs:91-105) rests on this."""
    g = torch.Generator(device="cuda").manual_seed(40 + epi)
    subs = [(0, 318), (318, 398), (716, 499), (1215, 263), (1741, 406)]
    t = 2147
    x = torch.randn(t, K, device="cuda", generator=g).to(BF16)
    n = 768 if epi == abi.EPI_RESID_F32 else 2304
    w = (torch.randn(n, K, device="cuda", generator=g) * 0.02).to(BF16)
    wp = hip.pack_ws(w)
    width = n // 2 if epi == abi.EPI_GEGLU_BF16 else n
    f32 = epi == abi.EPI_RESID_F32
    base = torch.randn(t, width, device="cuda", generator=g) if f32 else torch.zeros(t, width, dtype=BF16, device="cuda")
    pos = torch.randint(0, 8192, (t,), device="cuda", generator=g, dtype=torch.int32)
    cos, sin = (dev(v) for v in oracle.rope_table(10000.0, 8192))
    bias = torch.randn(n, device="cuda", generator=g) * 0.1

    def run(rows):
        out = base[rows].clone()
        kw = {}
        if epi == abi.EPI_ROPE_BF16:
            kw = dict(pos=pos[rows].contiguous(), cos=cos, sin=sin, rope_cols=1536)
        if epi == abi.EPI_BIAS_BF16:
            kw["bias"] = bias
        hip.op_gemm_ws(epi, x[rows].contiguous(), wp, n, K, out, **kw)
        return out

    full = run(slice(0, t))
    for s0, ln in subs:
        sub = run(slice(s0, s0 + ln))
        torch.cuda.synchronize()
        assert torch.equal(sub, full[s0:s0 + ln]), (s0, ln)


K2 = 1152


@pytest.mark.parametrize("rows,n", [(1, 768), (17, 768), (1000, 768), (9482, 768), (16384, 768), (30000, 768),
                                    (2000, 384), (9482, 384)])
def test_ws_k1152_residual(rows, n):
    """K = 1152 (Wo2 at hidden 768 and 384): one 16-token block, a partial block, ranges of 1 to 36 blocks, and
    more token blocks than ranges (30000 tokens: ~45 blocks per range)."""
    _case(rows, n, abi.EPI_RESID_F32, seed=rows + n, k=K2)


def test_ws_k1152_bias_stride_and_column_offset():
    _case(3001, 768, abi.EPI_RESID_F32, seed=5, bias=True, col=16, pad_out=8, ldx_pad=64, k=K2)


def test_ws_k1152_rows_independent_of_batch():
    """As test_ws_rows_independent_of_batch, for the K-split kernel."""
    g = torch.Generator(device="cuda").manual_seed(77)
    subs = [(0, 318), (318, 398), (716, 499), (1215, 263), (1741, 406)]
    t, n = 2147, 768
    x = torch.randn(t, K2, device="cuda", generator=g).to(BF16)
    w = (torch.randn(n, K2, device="cuda", generator=g) * 0.02).to(BF16)
    wp = hip.pack_ws(w)
    base = torch.randn(t, n, device="cuda", generator=g)

    def run(rows):
        out = base[rows].clone()
        hip.op_gemm_ws(abi.EPI_RESID_F32, x[rows].contiguous(), wp, n, K2, out)
        return out

    full = run(slice(0, t))
    for s0, ln in subs:
        sub = run(slice(s0, s0 + ln))
        torch.cuda.synchronize()
        assert torch.equal(sub, full[s0:s0 + ln]), (s0, ln)


def test_ws_k1152_rejects_other_epilogues():
    x = torch.zeros(64, K2, dtype=BF16, device="cuda")
    wp = hip.pack_ws(torch.zeros(768, K2, dtype=BF16))
    out = torch.zeros(64, 768, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError):
        hip.op_gemm_ws(abi.EPI_STORE_BF16, x, wp, 768, K2, out)
    with pytest.raises(hip.HipError):
        hip.pack_ws(torch.zeros(192, K2, dtype=BF16))


def test_pack_ws_layout_k1152():
    """At K = 1152: slab f (128 rows), wave w, slice s (of its K half), half h, lane l holds W row
    128f + 32(w % 4) + 16h + l % 16, K 32(18(w / 4) + s) + 8(l/16) .. +8."""
    n = 384
    w = torch.arange(n * K2, dtype=torch.int32).remainder(65521).to(torch.int16).view(BF16).reshape(n, K2)
    p = hip.pack_ws(w).cpu().view(torch.int16).numpy().reshape(n // 128, 8, 18, 2, 64, 8)
    src = w.view(torch.int16).numpy()
    rng = np.random.default_rng(6)
    for _ in range(300):
        f, wv, s = rng.integers(0, n // 128), rng.integers(0, 8), rng.integers(0, 18)
        h, ln = rng.integers(0, 2), rng.integers(0, 64)
        rw = 128 * f + 32 * (wv % 4) + 16 * h + ln % 16
        k0 = 32 * (18 * (wv // 4) + s) + 8 * (ln // 16)
        assert np.array_equal(p[f, wv, s, h, ln], src[rw, k0:k0 + 8])
