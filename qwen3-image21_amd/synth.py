"""Synthetic GGUF weights and block inputs for tests and the benchmark.

No checkpoint is available offline, so weights are drawn from N(0, std) and
quantized here into genuine GGML blocks (Q8_0, Q4_K, Q6_K). The quantizers are
plain fits (absmax for Q8_0/Q6_K, min/max for Q4_K); any valid block is a legal
input to the kernels, and the dequantization they are checked against is exact.
Generator: numpy.random.default_rng(seed); seeds are recorded by callers.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
BLOCK = {F32: (1, 4), F16: (1, 2), BF16: (1, 2), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210)}


def row_bytes(t: int, cols: int) -> int:
    bs, bb = BLOCK[t]
    assert cols % bs == 0
    return cols // bs * bb


def _round_half_away(v):
    v = np.asarray(v, dtype=np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def _f16_bits(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def _f16_val(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = _round_half_away((x * inv[:, None]).astype(np.float32)).astype(np.int8)
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = _f16_bits(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def quantize_q4_k(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).reshape(-1, 8, 32)
    nb = x.shape[0]
    mn = np.minimum(x.min(axis=2), 0).astype(np.float32)
    mx = x.max(axis=2).astype(np.float32)
    scales = ((mx - mn) / np.float32(15)).astype(np.float32)
    mins = (-mn).astype(np.float32)
    max_scale = scales.max(axis=1)
    max_min = mins.max(axis=1)
    inv_s = np.where(max_scale > 0, np.float32(63) / np.where(max_scale > 0, max_scale, 1), 0).astype(np.float32)
    inv_m = np.where(max_min > 0, np.float32(63) / np.where(max_min > 0, max_min, 1), 0).astype(np.float32)
    ls = np.clip(np.rint(inv_s[:, None] * scales), 0, 63).astype(np.uint8)
    lm = np.clip(np.rint(inv_m[:, None] * mins), 0, 63).astype(np.uint8)
    sc = np.zeros((nb, 12), dtype=np.uint8)
    sc[:, 0:4] = ls[:, 0:4] | ((ls[:, 4:8] >> 4) << 6)
    sc[:, 4:8] = lm[:, 0:4] | ((lm[:, 4:8] >> 4) << 6)
    sc[:, 8:12] = (ls[:, 4:8] & 0xF) | ((lm[:, 4:8] & 0xF) << 4)
    dbits = _f16_bits((max_scale / np.float32(63)).astype(np.float32))
    mbits = _f16_bits((max_min / np.float32(63)).astype(np.float32))
    d = _f16_val(dbits)
    dmin = _f16_val(mbits)
    ds = (d[:, None] * ls.astype(np.float32)).astype(np.float32)
    dm = (dmin[:, None] * lm.astype(np.float32)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        L = np.where(ds[:, :, None] != 0, np.rint((x + dm[:, :, None]) / np.where(ds != 0, ds, 1)[:, :, None]), 0)
    L = np.clip(L, 0, 15).astype(np.uint8).reshape(nb, 4, 2, 32)
    qs = (L[:, :, 0, :] | (L[:, :, 1, :] << 4)).reshape(nb, 128)
    out = np.empty((nb, 144), dtype=np.uint8)
    out[:, 0:2] = dbits.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = mbits.view(np.uint8).reshape(-1, 2)
    out[:, 4:16] = sc
    out[:, 16:] = qs
    return out.reshape(-1)


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32).reshape(-1, 16, 16)
    nb = x.shape[0]
    idx = np.abs(x).argmax(axis=2)
    mxv = np.take_along_axis(x, idx[:, :, None], axis=2)[:, :, 0]
    sub = np.where(np.abs(mxv) > 0, mxv / np.float32(-32), 0).astype(np.float32)
    j = np.abs(sub).argmax(axis=1)
    max_scale = sub[np.arange(nb), j]
    zero = np.abs(max_scale) == 0
    iscale = np.where(zero, 0, np.float32(-128) / np.where(zero, 1, max_scale)).astype(np.float32)
    scl = np.clip(np.rint(iscale[:, None] * sub), -128, 127).astype(np.int8)
    dbits = _f16_bits(np.where(zero, 0, np.float32(1) / np.where(zero, 1, iscale)).astype(np.float32))
    d = _f16_val(dbits)
    ds = (d[:, None] * scl.astype(np.float32)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(ds[:, :, None] != 0, np.rint(x / np.where(ds != 0, ds, 1)[:, :, None]), 0)
    L = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(nb, 2, 4, 32)  # [blk][half][r][l]
    ql = np.empty((nb, 2, 64), dtype=np.uint8)
    ql[:, :, 0:32] = (L[:, :, 0] & 0xF) | ((L[:, :, 2] & 0xF) << 4)
    ql[:, :, 32:64] = (L[:, :, 1] & 0xF) | ((L[:, :, 3] & 0xF) << 4)
    qh = (L[:, :, 0] >> 4) | ((L[:, :, 1] >> 4) << 2) | ((L[:, :, 2] >> 4) << 4) | ((L[:, :, 3] >> 4) << 6)
    out = np.empty((nb, 210), dtype=np.uint8)
    out[:, 0:128] = ql.reshape(nb, 128)
    out[:, 128:192] = qh.reshape(nb, 64)
    out[:, 192:208] = scl.view(np.uint8)
    out[:, 208:210] = dbits.view(np.uint8).reshape(-1, 2)
    return out.reshape(-1)


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if t == Q8_0:
        return quantize_q8_0(x)
    if t == Q4_K:
        return quantize_q4_k(x)
    if t == Q6_K:
        return quantize_q6_k(x)
    if t == F32:
        return x.reshape(-1).view(np.uint8).copy()
    if t == F16:
        return x.reshape(-1).astype(np.float16).view(np.uint8).copy()
    if t == BF16:
        u = x.reshape(-1).view(np.uint32).astype(np.uint64)
        b = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return b.view(np.uint8).copy()
    raise ValueError(t)


def random_blocks(rng, t: int, rows: int, cols: int, std: float = 0.02) -> np.ndarray:
    """Valid GGML blocks with uniformly random codes and scales sized for
    weights of standard deviation ~std; fast enough for checkpoint-sized
    benchmark weights (no quantization pass)."""
    nb = rows * cols // BLOCK[t][0]
    if t == Q8_0:
        out = rng.integers(0, 256, (nb, 34), dtype=np.uint8)
        out[:, 0:2] = _f16_bits(np.full(nb, std * 3.0 / 127.0 * 1.7)).view(np.uint8).reshape(-1, 2)
        return out.reshape(-1)
    if t == Q4_K:
        out = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
        out[:, 0:2] = _f16_bits(np.full(nb, std / 120.0)).view(np.uint8).reshape(-1, 2)
        out[:, 2:4] = _f16_bits(np.full(nb, std / 30.0)).view(np.uint8).reshape(-1, 2)
        return out.reshape(-1)
    if t == Q6_K:
        out = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
        out[:, 192:208] = rng.integers(-64, 65, (nb, 16)).astype(np.int8).view(np.uint8)
        out[:, 208:210] = _f16_bits(np.full(nb, std / 600.0)).view(np.uint8).reshape(-1, 2)
        return out.reshape(-1)
    return quantize(t, rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std))


def weight(rng, t: int, rows: int, cols: int, std: float = 0.02):
    """(type, bytes, rows, cols) of an N(0, std) weight [rows, cols] quantized to t."""
    w = (rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)).astype(np.float32)
    return (t, quantize(t, w), rows, cols)


def block_weights(seed: int, hidden: int, heads: int, mlp: int, attn_type: int = Q8_0,
                  down_type: int | None = None, fused_gate_up: bool = True, std: float = 0.02):
    """Weights of one block: to_q/k/v/out and gate_up (or proj + gate_layer) in attn_type,
    the MLP down projection in down_type, norm_q/norm_k = 1 + 0.02 N(0,1)."""
    rng = np.random.default_rng(seed)
    down_type = attn_type if down_type is None else down_type
    w = {}
    for n in ("to_q", "to_k", "to_v", "to_out"):
        w[n] = weight(rng, attn_type, hidden, hidden, std)
    if fused_gate_up:
        w["gate_up"] = weight(rng, attn_type, 2 * mlp, hidden, std)
    else:
        w["proj"] = weight(rng, attn_type, mlp, hidden, std)
        w["gate_layer"] = weight(rng, attn_type, mlp, hidden, std)
    w["down"] = weight(rng, down_type, hidden, mlp, std)
    hd = hidden // heads
    w["norm_q"] = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    w["norm_k"] = (1 + 0.02 * rng.standard_normal(hd)).astype(np.float32)
    return w


def weight_bytes(w: dict) -> int:
    return sum(v[1].size for k, v in w.items() if isinstance(v, tuple))


def t2i_layout(text_len: int, grid_h: int, grid_w: int):
    """Text-to-image joint layout facts: (image_mask, shapes) over text + target."""
    mask = [0] * text_len + [1] * (grid_h * grid_w)
    return mask, [(1, grid_h, grid_w)]
