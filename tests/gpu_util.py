"""Helpers shared by the GPU tests: device tensors and tolerance checks."""
import numpy as np
import torch


def dev(a, dtype=None):
    t = torch.as_tensor(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def bf16_round(a):
    """FP32 values rounded to bf16 (RNE) and widened back, on the CPU."""
    return torch.as_tensor(np.ascontiguousarray(a, dtype=np.float32)).bfloat16().float().numpy()


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()
