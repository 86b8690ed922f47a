"""jh_op_gemm_splitk_noalloc (the split-K GEMM whose FP32 partial sums live in
the library's fixed per-GPU scratch array) against jh_op_gemm_splitk (the same
kernels with a caller workspace), through the C-ABI: bit-identical outputs on
two calls in a row, the second with a smaller input, so stale partials of the
first call in the shared scratch cannot leak into the second.  Forced split
counts (which always use the scratch) and the automatic choice; a forced
split count whose partials exceed the scratch is rejected.
"""
import numpy as np
import pytest
import torch

from julia1_amd import abi, hip
from gpu_util import dev

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def _call(noalloc, epi, rows, n, k, splits, seed):
    r = np.random.default_rng(seed)
    x = dev(r.standard_normal((rows, k), dtype=np.float32), BF16)
    w = dev(r.standard_normal((n, k), dtype=np.float32) * 0.02, BF16)
    bias = dev(r.standard_normal(n, dtype=np.float32) * 0.1)
    if epi == abi.EPI_RESID_F32:
        out = dev(r.standard_normal((rows, n), dtype=np.float32))
    elif epi == abi.EPI_GEGLU_BF16:
        out = torch.zeros(rows, n // 2, dtype=BF16, device="cuda")
    else:
        out = torch.zeros(rows, n, dtype=BF16, device="cuda")
    kw = dict(bias=bias) if epi in (abi.EPI_RESID_F32, abi.EPI_BIAS_BF16) else {}
    if noalloc:
        hip.op_gemm_splitk_noalloc(epi, x, w, out, splits=splits, **kw)
    else:
        ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
        hip.op_gemm_splitk(epi, x, w, out, ws, splits=splits, **kw)
    torch.cuda.synchronize()
    return out.view(torch.int32 if out.dtype == torch.float32 else torch.int16).cpu().numpy()


@pytest.mark.parametrize("epi", [abi.EPI_RESID_F32, abi.EPI_STORE_BF16, abi.EPI_GEGLU_BF16, abi.EPI_BIAS_BF16])
@pytest.mark.parametrize("splits", [4, 0])
def test_noalloc_matches_workspace_entry(epi, splits):
    # first call larger, second smaller (fewer rows, narrower, shorter K)
    for i, (rows, n, k) in enumerate([(300, 768, 1152), (70, 384, 768)]):
        print(f"noalloc epi={epi} splits={splits} call={i} rows={rows} n={n} k={k}", flush=True)
        got = _call(True, epi, rows, n, k, splits, seed=100 + i)
        ref = _call(False, epi, rows, n, k, splits, seed=100 + i)
        assert got.shape == ref.shape and np.array_equal(got, ref), (epi, splits, rows, n, k)


def test_noalloc_rejects_partials_beyond_scratch():
    x = torch.zeros(4096, 768, dtype=BF16, device="cuda")
    w = torch.zeros(2304, 768, dtype=BF16, device="cuda")
    out = torch.zeros(4096, 2304, dtype=BF16, device="cuda")
    with pytest.raises(hip.HipError, match="exceed the 16 MiB scratch") as e:
        hip.op_gemm_splitk_noalloc(abi.EPI_STORE_BF16, x, w, out, splits=8)
    assert e.value.code == abi.JH_ERR_INVALID


_CAPTURE_CHILD = r"""
import sys
sys.path[:0] = [{root!r}, {pkg!r}]
import numpy as np
import torch
from julia1_amd import abi, hip

BF16 = torch.bfloat16
r = np.random.default_rng(7)
rows, n, k = 300, 768, 1152
x = torch.from_numpy(r.standard_normal((rows, k), dtype=np.float32)).cuda().to(BF16)
w = (torch.from_numpy(r.standard_normal((n, k), dtype=np.float32)) * 0.02).cuda().to(BF16)
bias = torch.from_numpy(r.standard_normal(n, dtype=np.float32) * 0.1).cuda()
out = torch.zeros(rows, n, dtype=BF16, device="cuda")
x2 = torch.from_numpy(r.standard_normal((70, 768), dtype=np.float32)).cuda().to(BF16)
w2 = (torch.from_numpy(r.standard_normal((384, 768), dtype=np.float32)) * 0.02).cuda().to(BF16)
out2 = torch.zeros(70, 384, dtype=BF16, device="cuda")
torch.cuda.synchronize()
print("capturing the library's first call", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    hip.op_gemm_splitk_noalloc(abi.EPI_BIAS_BF16, x, w, out, splits=4, bias=bias,
                               stream=torch.cuda.current_stream().cuda_stream)
ws = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
ref = torch.zeros_like(out)
hip.op_gemm_splitk(abi.EPI_BIAS_BF16, x, w, ref, ws, splits=4, bias=bias)
torch.cuda.synchronize()
for i in range(3):
    out.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), i
    # eager work between replays that rewrites the shared scratch with another call's partials
    hip.op_gemm_splitk_noalloc(abi.EPI_STORE_BF16, x2, w2, out2, splits=3)
    torch.cuda.synchronize()
print("replays match", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """In a fresh process, the library's first call is jh_op_gemm_splitk_noalloc captured by torch.cuda.graph on
    torch's capture stream (the scratch address is looked up during the capture); the graph is replayed three
    times, with an eager no-allocation call on another shape between replays, and every replay equals the
    workspace entry point's eager output bit for bit."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = _CAPTURE_CHILD.format(root=root, pkg=os.path.join(root, "julia1-rs_amd"))
    print("child: noalloc split-K GEMM captured as the first library call", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "replays match" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
