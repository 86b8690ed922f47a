"""C++ host engine (include/julia1_engine.h) checks that need no GPU: device
strings (src/engine.rs:20-32), the checkpoint reader's config/safetensors/
tensor-resolution paths and their error messages (src/config.rs:43-96,
src/weights.rs:51-89, src/model.rs:55-110, src/engine.rs:89-172)."""
import json
import os
import struct

import numpy as np
import pytest

from julia1_amd import engine, hip, synth


@pytest.fixture(scope="module")
def tiny_ckpt(tmp_path_factory):
    root = str(tmp_path_factory.mktemp("tiny"))
    cfg = synth.model_config("tiny")
    synth.write_checkpoint(root, "tiny", synth.make_weights(cfg, seed=1))
    return root


def test_parse_device():
    assert engine.parse_device("hip") == 0
    assert engine.parse_device("hip:3") == 3
    for bad in ("cpu", "cuda", "cuda:0", "hip:", "hip:x", "hip:-1", ""):
        with pytest.raises(hip.HipError, match="device must be hip or hip:N"):
            engine.parse_device(bad)


def test_inspect_reads_whole_checkpoint(tiny_ckpt):
    s = engine.inspect(tiny_ckpt)
    cfg = synth.model_config("tiny")
    assert s["hidden"] == 128 and s["layers"] == 3 and s["head_layers"] == 2
    assert s["tensors"] == len(synth.tensor_specs(cfg))
    assert s["bytes"] == os.path.getsize(os.path.join(tiny_ckpt, "model.safetensors"))


def _copy_ckpt(src, dst, julia=None, enc=None, weights=None):
    os.makedirs(os.path.join(dst, "encoder"), exist_ok=True)
    j = json.load(open(os.path.join(src, "julia_config.json")))
    e = json.load(open(os.path.join(src, "encoder", "config.json")))
    j.update(julia or {})
    e.update(enc or {})
    json.dump(j, open(os.path.join(dst, "julia_config.json"), "w"))
    json.dump(e, open(os.path.join(dst, "encoder", "config.json"), "w"))
    if weights is None:
        os.symlink(os.path.join(src, "model.safetensors"), os.path.join(dst, "model.safetensors"))
    else:
        open(os.path.join(dst, "model.safetensors"), "wb").write(weights)
    return dst


@pytest.mark.parametrize("julia,enc,msg", [
    ({"format_version": 2}, {}, "Unsupported Julia checkpoint format"),
    ({"weight_dtype": "int8"}, {}, "Only float32 Julia checkpoints are supported"),
    ({}, {"model_type": "bert"}, "Encoder must be ModernBERT"),
    ({}, {"norm_bias": True}, "Unsupported encoder setting norm_bias"),
    ({}, {"hidden_activation": "relu"}, "Unsupported encoder activation"),
    ({}, {"num_attention_heads": 4}, "Runtime kernels require head_dim 64"),
    ({}, {"layer_types": ["full_attention"]}, "layer_types must list every layer"),
    ({}, {"rope_parameters": {"full_attention": {"rope_type": "yarn", "rope_theta": 1.0}}}, "Only default RoPE"),
    ({"head_layers": None}, {}, "config is missing head_layers"),
])
def test_config_errors(tiny_ckpt, tmp_path, julia, enc, msg):
    d = _copy_ckpt(tiny_ckpt, str(tmp_path / "c"), julia, enc)
    with pytest.raises(hip.HipError, match=msg):
        engine.inspect(d)


def _safetensors(tensors, dtype="F32"):
    header, blobs, off = {}, [], 0
    for name, a in tensors.items():
        b = a.astype(np.float32 if dtype == "F32" else np.float16).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + b"".join(blobs)


def test_safetensors_errors(tiny_ckpt, tmp_path):
    cases = [
        (b"version https://git-lfs.github.com/spec/v1\noid sha256:00\nsize 1\n", "Git LFS pointers"),
        (b"\x01\x02", "Truncated safetensors file"),
        (struct.pack("<Q", 1 << 40) + b"{}", "Truncated safetensors header"),
        (_safetensors({"x": np.zeros(3)}, dtype="F16"), "only F32 tensors are supported"),
        (_safetensors({"x": np.zeros(3)}), "missing tensor encoder.embeddings.tok_embeddings.weight"),
    ]
    for i, (blob, msg) in enumerate(cases):
        d = _copy_ckpt(tiny_ckpt, str(tmp_path / f"s{i}"), weights=blob)
        with pytest.raises(hip.HipError, match=msg):
            engine.inspect(d)


def _raw_header(header: dict, data: bytes = b"") -> bytes:
    h = json.dumps(header).encode()
    return struct.pack("<Q", len(h)) + h + data


@pytest.mark.parametrize("offsets", [
    [0, 2 ** 64 - 1],                       # end near 2^64: 8 + n + end would wrap
    [2 ** 64 - 16, 2 ** 64 - 4],            # both near 2^64
    [0, 2 ** 64],                           # beyond u64
    [0, 2 ** 53 + 1],                       # above double precision: must not round into range
    [12, 4],                                # begin after end
    [0, 13],                                # one past the data
])
def test_safetensors_offsets_out_of_range(tiny_ckpt, tmp_path, offsets):
    """data_offsets are read exactly from their literal text and bounds-checked without wrap-around
    (the reference slices the mapping with checked bounds, src/weights.rs:79-89)."""
    blob = _raw_header({"x": {"dtype": "F32", "shape": [3], "data_offsets": offsets}}, b"\0" * 12)
    d = _copy_ckpt(tiny_ckpt, str(tmp_path / "o"), weights=blob)
    with pytest.raises(hip.HipError, match="data out of bounds|data_offsets"):
        engine.inspect(d)


def test_wrong_tensor_shape(tmp_path):
    cfg = synth.model_config("tiny")
    t = synth.make_weights(cfg, seed=2)
    t["encoder.layers.1.mlp.Wo.weight"] = np.zeros((128, 100), dtype=np.float32)
    d = synth.write_checkpoint(str(tmp_path / "w"), "tiny", t)
    with pytest.raises(hip.HipError, match=r"encoder.layers.1.mlp.Wo.weight: expected shape \[128, 192\], found \[128, 100\]"):
        engine.inspect(d)


def test_load_option_errors_before_any_device(tiny_ckpt, tmp_path):
    with pytest.raises(hip.HipError, match="max_length must be an integer between 1 and 256"):
        engine.Engine.load(tiny_ckpt, max_length=257)
    with pytest.raises(hip.HipError, match="Invalid batch size / token budget"):
        engine.Engine.load(tiny_ckpt, batch_size=0)
    with pytest.raises(hip.HipError, match="Invalid batch size / token budget"):
        engine.Engine.load(tiny_ckpt, max_batch_tokens=100)
    d = _copy_ckpt(tiny_ckpt, str(tmp_path / "q"))
    open(os.path.join(d, "quantization.json"), "w").write("{}")
    with pytest.raises(hip.HipError, match="INT8 checkpoints are not supported"):
        engine.Engine.load(d)


def test_load_without_gpu_fails_cleanly(tiny_ckpt):
    torch = pytest.importorskip("torch")
    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present; covered by the GPU tests")
    with pytest.raises(hip.HipError) as e:
        engine.Engine.load(tiny_ckpt)
    assert e.value.code == 2


def test_bf16_rounding_matches_torch():
    """checkpoint.bf16_bits against torch's FP32 -> BF16 conversion (round to
    nearest even), on random values and the tie/overflow/NaN special cases."""
    torch = pytest.importorskip("torch")
    from julia1_amd import checkpoint
    rng = np.random.default_rng(5)
    u = np.concatenate([rng.integers(0, 2**32, 100000, dtype=np.uint64).astype(np.uint32),
                        np.array([0x3F808000, 0x3F818000, 0x3F807FFF, 0x7F7FFFFF, 0xFF7FFFFF, 0x7F800000,
                                  0x00008000, 0x00018000, 0x80000000], dtype=np.uint32)])
    a = u.view(np.float32)
    finite = np.isfinite(a)
    got = checkpoint.bf16_bits(a)
    want = torch.from_numpy(a.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[finite], want[finite])
    assert got[-9] == 0x3F80 and got[-8] == 0x3F82 and got[-7] == 0x3F80 and got[-6] == 0x7F80
    nan = np.isnan(a)
    assert np.isnan(checkpoint.bf16_to_f32(got[nan])).all()
    assert np.array_equal(checkpoint.bf16_to_f32(got[finite]).view(np.uint32),
                          want[finite].astype(np.uint32) << np.uint32(16))


@pytest.fixture(scope="module")
def bf16_ckpt(tiny_ckpt, tmp_path_factory):
    from julia1_amd import checkpoint
    return checkpoint.convert_to_bf16(tiny_ckpt, str(tmp_path_factory.mktemp("bf16")))


def test_bf16_checkpoint_layout(tiny_ckpt, bf16_ckpt):
    """The converted file reads back through the safetensors library itself:
    matrices as torch's BF16 rounding of the F32 originals, the rest unchanged."""
    torch = pytest.importorskip("torch")
    from safetensors.torch import load_file
    from julia1_amd import checkpoint
    src = load_file(os.path.join(tiny_ckpt, "model.safetensors"))
    dst = load_file(os.path.join(bf16_ckpt, "model.safetensors"))
    assert src.keys() == dst.keys()
    n_bf16 = 0
    for name, a in src.items():
        b = dst[name]
        if checkpoint.is_bf16_matrix(name):
            n_bf16 += 1
            assert b.dtype == torch.bfloat16 and torch.equal(b, a.to(torch.bfloat16))
        else:
            assert b.dtype == torch.float32 and torch.equal(a, b)
    cfg = synth.model_config("tiny")
    assert n_bf16 == 4 * cfg.layers + 4 * cfg.head_layers + 1
    assert json.load(open(os.path.join(bf16_ckpt, "julia_config.json")))["weight_dtype"] == "bfloat16"
    s = engine.inspect(bf16_ckpt)
    assert s["tensors"] == len(src) and s["bf16_tensors"] == n_bf16
    assert engine.inspect(tiny_ckpt)["bf16_tensors"] == 0
    assert s["bytes"] < 0.75 * os.path.getsize(os.path.join(tiny_ckpt, "model.safetensors"))


def test_bf16_checkpoint_errors(tiny_ckpt, bf16_ckpt, tmp_path):
    from julia1_amd import checkpoint
    # BF16 tensors under weight_dtype float32: the reference's F32-only rule.
    d = _copy_ckpt(bf16_ckpt, str(tmp_path / "a"), julia={"weight_dtype": "float32"})
    with pytest.raises(hip.HipError, match="only F32 tensors are supported"):
        engine.inspect(d)
    # bfloat16 checkpoints accept F32 and BF16, nothing else.
    d = _copy_ckpt(tiny_ckpt, str(tmp_path / "b"), julia={"weight_dtype": "bfloat16"},
                   weights=_safetensors({"x": np.zeros(3)}, dtype="F16"))
    with pytest.raises(hip.HipError, match="only F32 and BF16 tensors are supported"):
        engine.inspect(d)
    # An all-F32 file is a valid bfloat16 checkpoint.
    d = _copy_ckpt(tiny_ckpt, str(tmp_path / "c"), julia={"weight_dtype": "bfloat16"})
    assert engine.inspect(d)["bf16_tensors"] == 0
    # A tensor whose shape, or whose byte length, disagrees with what the model needs.
    cfg = synth.model_config("tiny")
    t = synth.make_weights(cfg, seed=3)
    name = "encoder.layers.0.attn.Wo.weight"
    p = str(tmp_path / "d.safetensors")
    checkpoint.write_safetensors(p, {k: (("BF16", checkpoint.bf16_bits(v)) if k == name else v) for k, v in t.items()})
    blob = open(p, "rb").read()
    n = int.from_bytes(blob[:8], "little")
    data = blob[8 + n:]

    def with_header(edit, sub):
        header = json.loads(blob[8:8 + n])
        edit(header[name])
        h = json.dumps(header).encode()
        h += b" " * (-len(h) % 8)
        return _copy_ckpt(tiny_ckpt, str(tmp_path / sub), julia={"weight_dtype": "bfloat16"},
                          weights=len(h).to_bytes(8, "little") + h + data)

    assert engine.inspect(with_header(lambda e: None, "e"))["bf16_tensors"] == 1
    with pytest.raises(hip.HipError, match=r"attn.Wo.weight: expected shape \[128, 128\], found \[128, 64\]"):
        engine.inspect(with_header(lambda e: e.update(shape=[128, 64]), "f"))
    with pytest.raises(hip.HipError, match="attn.Wo.weight: data length does not match its shape"):
        engine.inspect(with_header(lambda e: e.update(data_offsets=[e["data_offsets"][0], e["data_offsets"][1] - 2]), "g"))
