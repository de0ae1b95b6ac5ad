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


def check_block(got, cand, exact, x):
    """A block output against the oracle's candle mode (cand) and exact mode
    (exact) on the same token rows [R, hidden]; x: their inputs. Against exact
    arithmetic: cosine >= 0.9999 on the output and on the update, and
    max|a-b|/max|b| <= 2e-2; the GPU lies at least as close to exact arithmetic
    as the candle path does; against the candle path: max|a-b|/max|b| <= 2e-2
    and a cosine no lower than the candle path's own to exact arithmetic (less
    2e-5), capped at 0.9999. The cap matters at MLP 12288, where the int8
    quantization of the SwiGLU hidden state alone puts the candle output at
    cosine ~0.99988 from exact arithmetic."""
    c_ge, c_ce = cos_sim(got, exact), cos_sim(cand, exact)
    u_ge, u_ce = cos_sim(got - x, exact - x), cos_sim(cand - x, exact - x)
    c_gc = cos_sim(got, cand)
    print(f"cos(gpu, exact) {c_ge:.7f} update {u_ge:.7f}; cos(candle, exact) {c_ce:.7f} update {u_ce:.7f}; "
          f"cos(gpu, candle) {c_gc:.7f}; mar gpu-exact {max_abs_rel(got, exact):.2e} "
          f"gpu-candle {max_abs_rel(got, cand):.2e}", flush=True)
    assert c_ge >= 0.9999 and u_ge >= 0.9999 and max_abs_rel(got, exact) <= 2e-2
    assert c_ge >= c_ce and u_ge >= u_ce        # closer to exact arithmetic than the candle path
    assert c_gc >= min(0.9999, c_ce - 2e-5) and max_abs_rel(got, cand) <= 2e-2
