"""Host-side checks that need no GPU: the C-ABI library loads and exports
every function include/*.h declares; the config parser restates
ModelConfig::from_values; the synthetic generators are deterministic."""
import json
import os
import re

import numpy as np
import pytest

from julia1_amd import abi, hip, synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for f in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if f.endswith(".h"):
            text = open(os.path.join(ROOT, "include", f)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names += re.findall(r"^\s*(?:const\s+)?[\w]+\s*\**\s*(j[het]_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 20
    lib = hip.lib()
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(hip.EXPORTS) <= set(names)
    from julia1_amd import text
    assert set(text.EXPORTS) <= set(names)


def test_static_archive_exports_every_declared_symbol():
    """libjulia1_hip.a (the archive a Rust build.rs links) defines every function include/*.h declares, and the
    C99 caller under tests/c_abi was linked against it (not against the shared object)."""
    import subprocess
    from julia1_amd import build_paths
    out = subprocess.run(["nm", "-g", "--defined-only", build_paths.ARCHIVE], capture_output=True, text=True, check=True)
    defined = set(re.findall(r" T (j[het]_\w+)$", out.stdout, flags=re.M))
    missing = [n for n in declared_functions() if n not in defined]
    assert not missing, missing
    assert os.access(build_paths.CALLER, os.X_OK)
    deps = subprocess.run(["ldd", build_paths.CALLER], capture_output=True, text=True).stdout
    assert "libjulia1_hip" not in deps and "libamdhip64" in deps, deps


def test_last_error_is_empty_string_initially():
    assert hip.lib().jh_last_error() is not None


def test_create_without_device_reports_error_not_crash():
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present; covered by the GPU tests")
    cfg = synth.model_config("tiny")
    ws = abi.WeightSet(cfg, synth.make_weights(cfg, 0))
    with pytest.raises(hip.HipError) as e:
        hip.HipModel(ws)
    assert e.value.code == 2


def test_create_rejects_bad_config_before_touching_device():
    cfg = synth.model_config("tiny")
    ws = abi.WeightSet(cfg, synth.make_weights(cfg, 0))
    ws.config.head_dim = 32
    with pytest.raises(hip.HipError) as e:
        hip.HipModel(ws)
    assert e.value.code == 1


def test_config_from_values_base():
    c = synth.model_config("modernbert-base")
    assert (c.hidden, c.heads, c.head_dim, c.intermediate, c.layers) == (768, 12, 64, 1152, 22)
    assert c.global_ == [i % 3 == 0 for i in range(22)] and sum(c.global_) == 8
    assert c.half_window == 64 and c.head_ff == 3072 and c.head_heads == 12
    assert c.rope_theta == [160000.0 if i % 3 == 0 else 10000.0 for i in range(22)]


def test_config_rejections():
    s = synth.SHAPES["tiny"]
    for key, val in (("hidden_activation", "relu"), ("norm_bias", True), ("model_type", "bert")):
        enc = dict(s["enc"], **{key: val})
        with pytest.raises(ValueError):
            abi.ModelConfig.from_values(s["julia"], enc)
    with pytest.raises(ValueError):
        abi.ModelConfig.from_values(dict(s["julia"], format_version=2), s["enc"])
    with pytest.raises(ValueError):
        abi.ModelConfig.from_values(dict(s["julia"], weight_dtype="int8"), s["enc"])
    enc = dict(s["enc"], hidden_size=96, num_attention_heads=2)
    with pytest.raises(ValueError):
        abi.ModelConfig.from_values(s["julia"], enc)


def test_rope_parameters_override():
    s = synth.SHAPES["tiny"]
    enc = dict(s["enc"], rope_parameters={"full_attention": {"rope_type": "default", "rope_theta": 5e5},
                                          "sliding_attention": {"rope_type": "default", "rope_theta": 2e4}})
    c = abi.ModelConfig.from_values(s["julia"], enc)
    assert c.rope_theta == [5e5, 2e4, 2e4]


def test_workloads_are_deterministic_and_shaped():
    b1 = synth.workload("config1")
    b1b = synth.workload("config1")
    assert np.array_equal(b1.ids, b1b.ids) and np.array_equal(b1.marker_rows, b1b.marker_rows)
    assert b1.lens.size == 32 and b1.lens.min() >= 64 and b1.lens.max() <= 512
    opts = np.diff(b1.marker_starts)
    assert opts.min() >= 2 and opts.max() <= 20
    assert b1.ids.max() < 50368
    b4 = synth.workload("config4")
    assert b4.lens.size == 256 and 32 <= b4.lens.min() and b4.lens.max() <= 1024
    assert 120_000 < b4.tokens < 150_000 and b4.marker_rows.size == 5120
    for b in (b1, b4):
        for s in range(b.lens.size):
            rows = b.marker_rows[b.marker_starts[s]:b.marker_starts[s + 1]]
            assert np.all((rows >= b.starts[s]) & (rows < b.starts[s] + b.lens[s]))


def test_padded_round_trip():
    b = synth.workload("config1").subset(range(5))
    ids, lens, qt, markers, mst = synth.padded(b, 512)
    assert ids.shape == (5, 512)
    for s in range(5):
        assert np.array_equal(ids[s, :lens[s]], b.ids[b.starts[s]:b.starts[s] + lens[s]])


def test_interleave_geglu_layout():
    inter, k = 96, 5
    wi = np.arange(2 * inter * k, dtype=np.float32).reshape(2 * inter, k)
    out = hip.interleave_geglu(wi)
    for j in range(inter // 32):
        assert np.array_equal(out[64 * j:64 * j + 32], wi[32 * j:32 * j + 32])
        assert np.array_equal(out[64 * j + 32:64 * j + 64], wi[inter + 32 * j:inter + 32 * j + 32])


def _build_module():
    import importlib.util
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "julia1-rs_amd", "build.py")
    spec = importlib.util.spec_from_file_location("jh_build", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_kernel_resource_remarks_parsed_and_scratch_rejected():
    """The build reads each kernel's figures from hipcc's kernel-resource-usage remarks and fails on any
    kernel with per-lane scratch."""
    b = _build_module()
    text = "\n".join([
        "x.hip:10:1: remark: Function Name: _Z3fooPf [-Rpass-analysis=kernel-resource-usage]",
        "   10 | __global__ void foo(float* p) {",
        "      | ^",
        "x.hip:10:1: remark:     VGPRs: 24 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:10:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:10:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:10:1: remark:     LDS Size [bytes/block]: 4096 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:20:1: remark: Function Name: _Z3barPf [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:20:1: remark:     VGPRs: 40 [-Rpass-analysis=kernel-resource-usage]",
        "x.hip:20:1: remark:     ScratchSize [bytes/lane]: 52 [-Rpass-analysis=kernel-resource-usage]",
    ])
    r = b.kernel_resources(text)
    assert r == {"_Z3fooPf": {"vgprs": 24, "agprs": 0, "scratch": 0, "lds": 4096},
                 "_Z3barPf": {"vgprs": 40, "scratch": 52}}
    b.check_no_scratch({"_Z3fooPf": r["_Z3fooPf"]})
    with pytest.raises(RuntimeError, match="_Z3barPf"):
        b.check_no_scratch(r)


def test_built_kernels_use_no_scratch():
    """The figures the last build recorded: every kernel of the library (the GEMMs, attention, the row
    kernels) runs without per-lane scratch memory."""
    b = _build_module()
    if not os.path.exists(b.RESOURCES):
        pytest.skip("library not built here")
    with open(b.RESOURCES) as f:
        res = json.load(f)
    names = " ".join(res)
    for k in ("gemm_ws_kernel", "gemm_big_kernel", "resid_reduce_ln_kernel", "layer_norm_kernel", "attention_kernel"):
        assert k in names, k
    assert all(v.get("scratch") == 0 for v in res.values()), {k: v for k, v in res.items() if v.get("scratch")}
