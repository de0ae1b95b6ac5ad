"""Helpers for the GPU parity tests: device buffers through torch, metrics of
the reference's probes (src/bin/quant_vs_full_probe.rs:13-17,
src/bin/kv_cache_probe.rs:11-14)."""
import numpy as np


def cos_sim(a, b):
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


def max_abs_rel(a, b):
    """max|a - b| / max|b| (b = reference)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def dev(torch, arr):
    return torch.from_numpy(np.ascontiguousarray(arr)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bf16_dev(torch, x_f32):
    """f32 numpy -> bf16 device tensor (round to nearest even), plus its f32 value."""
    t = torch.from_numpy(np.ascontiguousarray(x_f32, dtype=np.float32)).to(torch.bfloat16)
    return t.cuda(), t.float().numpy()


def stream(torch):
    return torch.cuda.current_stream().cuda_stream
