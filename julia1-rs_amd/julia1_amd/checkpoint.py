"""BF16 checkpoints for the HIP engine.

The reference reads F32 safetensors only (src/weights.rs:64) and rounds every
weight matrix to BF16 when it uploads it (half::bf16::from_f32, round to
nearest even; src/cuda/mod.rs:36-39,204-262).  `convert_to_bf16` writes that
rounding to disk once: the matrices become BF16 tensors, everything the backend
keeps in FP32 (embedding, norms, biases, type_emb, scorer.3) stays F32, and
julia_config.json says weight_dtype "bfloat16".  The engine widens a BF16
tensor to FP32 exactly and the backend's rounding of an already-BF16 value is
the identity, so such a checkpoint yields the same device weights, and hence
the same logits bit for bit, as the F32 checkpoint it came from, at about half
the file size.
"""
import json
import os
import shutil

import numpy as np

# Tensor-name suffixes of the matrices the backend stores as BF16
# (src/cuda/mod.rs:204-262: Wqkv, Wo, Wi, mlp Wo, head in/out projections,
# linear1/2 and scorer.1).
BF16_MATRICES = ("attn.Wqkv.weight", "attn.Wo.weight", "mlp.Wi.weight", "mlp.Wo.weight",
                 "self_attn.in_proj_weight", "self_attn.out_proj.weight", "linear1.weight",
                 "linear2.weight", "scorer.1.weight")


def is_bf16_matrix(name: str) -> bool:
    return name.endswith(BF16_MATRICES)


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """FP32 -> BF16 bit patterns, round to nearest even; NaN stays a quiet NaN."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    rounded = ((u + (np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1)))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, ((u >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16), rounded)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def write_safetensors(path: str, tensors: dict) -> None:
    """tensors: name -> float32 ndarray (stored F32) or ("BF16", uint16 ndarray).

    Layout per the safetensors format: u64 little-endian header length, the
    JSON header (padded with spaces to a multiple of 8), then the raw
    little-endian data in header order.
    """
    header, blobs, off = {}, [], 0
    for name, t in tensors.items():
        if isinstance(t, tuple):
            dtype, a = t
            if dtype != "BF16" or a.dtype != np.uint16:
                raise ValueError(f"{name}: BF16 tensors are given as uint16 bit patterns")
        else:
            dtype, a = "F32", np.asarray(t, dtype=np.float32)
        b = np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def convert_to_bf16(src: str, dst: str, all_tensors: bool = False) -> str:
    """Write a weight_dtype "bfloat16" copy of the F32 checkpoint directory `src` to `dst`.

    all_tensors=True also stores the FP32-resident tensors as BF16 (a smaller
    file whose logits then differ from the F32 checkpoint's by that rounding).
    """
    from safetensors.numpy import load_file  # no code execution: raw tensor data only

    with open(os.path.join(src, "julia_config.json")) as f:
        julia = json.load(f)
    if julia.get("weight_dtype", "float32") != "float32":
        raise ValueError("source checkpoint must be float32")
    tensors = load_file(os.path.join(src, "model.safetensors"))
    out = {}
    for name, a in tensors.items():
        if a.dtype != np.float32:
            raise ValueError(f"{name}: only F32 tensors are supported")
        out[name] = ("BF16", bf16_bits(a)) if all_tensors or is_bf16_matrix(name) else a
    os.makedirs(os.path.join(dst, "encoder"), exist_ok=True)
    julia["weight_dtype"] = "bfloat16"
    with open(os.path.join(dst, "julia_config.json"), "w") as f:
        json.dump(julia, f)
    shutil.copyfile(os.path.join(src, "encoder", "config.json"), os.path.join(dst, "encoder", "config.json"))
    write_safetensors(os.path.join(dst, "model.safetensors"), out)
    return dst
