"""ctypes wrapper of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the CPU
baseline leg of bench.py, never by the product library. numpy in, numpy out.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q8_0, Q4_K, Q6_K, Q8_K, BF16 = 0, 1, 8, 12, 14, 15, 30
CANDLE, EXACT = 0, 1

_lib = None


NATIVE_PATH = os.path.join(HERE, "_native", "liboracle_native.so")
_isa = "x86-64-v3"


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def use_native_build():
    """Build the oracle for this host's own instruction set (-march=native,
    always rebuilt here, never a copy made on another machine) and load it in
    place of the portable x86-64-v3 build; for the timed CPU baseline. Must run
    before the first lib() call. Returns the ISA label of the loaded build."""
    global LIB_PATH, _isa
    if _lib is not None:
        return _isa
    try:
        subprocess.run(["make", "-s", "-B", "-C", HERE, "native"], check=True, capture_output=True, timeout=300)
        LIB_PATH, _isa = NATIVE_PATH, "native"
    except (OSError, subprocess.SubprocessError):
        pass
    return _isa


def isa():
    return _isa


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "oq_f16_to_f32": (C.c_float, [C.c_uint16]),
            "oq_f32_to_f16": (C.c_uint16, [C.c_float]),
            "oq_bf16_to_f32": (C.c_float, [C.c_uint16]),
            "oq_f32_to_bf16": (C.c_uint16, [C.c_float]),
            "oq_f32_to_bf16_n": (None, [vp, i64, vp]),
            "oq_bf16_to_f32_n": (None, [vp, i64, vp]),
            "oq_block_size": (i32, [i32]),
            "oq_block_bytes": (i32, [i32]),
            "oq_row_bytes": (i64, [i32, i64]),
            "oq_quantize": (i32, [i32, vp, i64, vp]),
            "oq_quant_act_bf16": (i32, [i32, vp, i64, i64, vp]),
            "oq_dequantize": (i32, [i32, vp, i64, vp]),
            "oq_qmatmul": (i32, [i32, vp, i64, i64, vp, i64, vp, i32]),
            "oq_layernorm_mod": (None, [vp, i64, i64, vp, i64, i64, C.c_float, vp]),
            "oq_rmsnorm": (None, [vp, i64, i64, vp, C.c_float]),
            "oq_rope_table": (i32, [vp, i32, vp, i64, vp, C.c_double, vp]),
            "oq_apply_rope": (None, [vp, i64, i64, i64, vp]),
            "oq_joint_layout": (i32, [i64, vp, vp, i32, i64, i64, vp, i64, vp, vp, vp]),
            "oq_block_causal_mask": (None, [vp, i64, vp]),
            "oq_attention": (i32, [vp, vp, vp, i64, vp, vp, i64, i64, i64, i64, i64, C.c_double, vp, i64, vp, i32]),
            "oq_block_forward": (i32, [vp, vp, vp, i64, i64, vp, i64, vp, vp, i64, vp, vp, i64, vp, vp, vp, i32]),
            "oq_block_forward_rows": (i32, [vp, vp, vp, i64, i64, vp, i64, vp, vp, i64, vp, vp, i64, vp, i64,
                                            vp, vp, vp, i32]),
            "oq_timestep_embedding": (None, [vp, i64, i64, vp]),
            "oq_silu_inplace": (None, [vp, i64]),
            "oq_now_seconds": (C.c_double, []),
            "oq_num_threads": (i32, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- conversions ----
def f32_to_bf16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oq_f32_to_bf16_n(_p(x), x.size, _p(out))
    return out


def bf16_to_f32(b):
    b = _c(b, np.uint16)
    out = np.empty(b.shape, dtype=np.float32)
    lib().oq_bf16_to_f32_n(_p(b), b.size, _p(out))
    return out


def bf16_round(x):
    return bf16_to_f32(f32_to_bf16(x))


# ---- codecs ----
def row_bytes(t, n):
    return int(lib().oq_row_bytes(t, n))


def quantize(t, x):
    """x [..., K] f32 -> GGUF block bytes (uint8 array, rows concatenated)."""
    x = _c(x, np.float32)
    nb = row_bytes(t, x.shape[-1])
    if nb < 0:
        raise ValueError("size is not a block multiple")
    out = np.empty(x.size // x.shape[-1] * nb, dtype=np.uint8)
    rc = lib().oq_quantize(t, _p(x), x.size, _p(out))
    assert rc == 0
    return out


def dequantize(t, data, n):
    data = _c(data, np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib().oq_dequantize(t, _p(data), n, _p(out))
    assert rc == 0
    return out


def quant_act_bf16(wtype, x):
    """candle's activation rounding of the rows of x [..., K] for a wtype weight
    (Q8_0 / Q4_K / Q6_K), as the bf16 bits of d * q (uint16, same shape)."""
    x = _c(x, np.float32)
    k = x.shape[-1]
    out = np.empty(x.shape, dtype=np.uint16)
    rc = lib().oq_quant_act_bf16(wtype, _p(x), x.size // k, k, _p(out))
    assert rc == 0, rc
    return out


# ---- GEMM ----
def qmatmul(t, w, n, k, x, mode=CANDLE):
    x = _c(x, np.float32)
    m = x.size // k
    y = np.empty((m, n), dtype=np.float32)
    w = _c(w, np.uint8)
    rc = lib().oq_qmatmul(t, _p(w), n, k, _p(x), m, _p(y), mode)
    assert rc == 0, rc
    return y


# ---- row ops ----
def layernorm_mod(x, scale=None, eps=1e-6):
    x = _c(x, np.float32)
    rows, cols = x.size // x.shape[-1], x.shape[-1]
    out = np.empty_like(x)
    sc = None if scale is None else _c(scale, np.float32)
    lib().oq_layernorm_mod(_p(x), rows, cols, _p(sc), 0, max(rows, 1), eps, _p(out))
    return out


def rmsnorm(x, w, eps=1e-6):
    x = _c(x, np.float32).copy()
    w = _c(w, np.float32)
    lib().oq_rmsnorm(_p(x), x.size // x.shape[-1], x.shape[-1], _p(w), eps)
    return x


def rope_table(shapes, image_mask, axes=(16, 56, 56), theta=10000.0):
    seq = len(image_mask)
    pe = np.zeros((seq, int(sum(axes))), dtype=np.float32)
    sh = np.array([v for s in shapes for v in s], dtype=np.int64)
    m = np.array([1 if v else 0 for v in image_mask], dtype=np.uint8)
    ax = np.array(axes, dtype=np.int64)
    rc = lib().oq_rope_table(_p(sh) if len(sh) else None, len(shapes), _p(m) if seq else None, seq,
                             _p(ax), theta, _p(pe) if seq else None)
    if rc != 0:
        raise ValueError(f"oq_rope_table -> {rc}")
    return pe


def apply_rope(x, pe):
    """x [..., S, D] rotated by pe [S, D]."""
    x = _c(x, np.float32).copy()
    s, d = x.shape[-2], x.shape[-1]
    pe = _c(pe, np.float32)
    lib().oq_apply_rope(_p(x), x.size // (s * d), s, d, _p(pe))
    return x


def joint_layout(text_len, text_image_mask=None, cond_shapes=(), target=(1, 1)):
    cap = text_len * 8 + sum(h * w for h, w in cond_shapes) + target[0] * target[1] + 16
    ids = np.zeros(cap, dtype=np.int64)
    m = None if text_image_mask is None else np.array([1 if v else 0 for v in text_image_mask] or [0], np.uint8)
    cs = np.array([v for hw in cond_shapes for v in hw] or [0], dtype=np.int64)
    pl, tl, tot = C.c_int64(), C.c_int64(), C.c_int64()
    rc = lib().oq_joint_layout(text_len, _p(m), _p(cs), len(cond_shapes), target[0], target[1], _p(ids), cap,
                               C.byref(pl), C.byref(tl), C.byref(tot))
    if rc != 0:
        raise ValueError(f"oq_joint_layout -> {rc}")
    return ids[: tot.value].tolist(), pl.value, tl.value


def block_causal_mask(image_ids):
    ids = _c(image_ids, np.int64)
    s = ids.size
    m = np.zeros((s, s), dtype=np.uint8)
    lib().oq_block_causal_mask(_p(ids), s, _p(m))
    return m


# ---- attention ----
def attention(q, k_own, v_own, k_pre=None, v_pre=None, scale=None, mask=None, mode=CANDLE):
    """q [B,H,Sq,D]; k/v own [B,H,So,D]; optional prefix [B,H,P,D]; mask [B|1,Sq,P+So]."""
    q = _c(q, np.float32)
    b, h, sq, d = q.shape
    ko, vo = _c(k_own, np.float32), _c(v_own, np.float32)
    so = ko.shape[2]
    p = 0
    kp = vp = None
    if k_pre is not None:
        kp, vp = _c(k_pre, np.float32), _c(v_pre, np.float32)
        p = kp.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(d)
    mk, mstride = None, 0
    if mask is not None:
        mk = _c(mask, np.uint8)
        mstride = 0 if mk.shape[0] == 1 else sq * (p + so)
    out = np.empty_like(q)
    rc = lib().oq_attention(_p(q), _p(kp), _p(vp), p, _p(ko), _p(vo), so, b, h, sq, d, float(scale), _p(mk),
                            mstride, _p(out), mode)
    assert rc == 0
    return out


# ---- block ----
class _QW(C.Structure):
    _fields_ = [("type", C.c_int), ("data", C.c_void_p), ("rows", C.c_int64), ("cols", C.c_int64)]


class _BW(C.Structure):
    _fields_ = [("to_q", _QW), ("to_k", _QW), ("to_v", _QW), ("to_out", _QW), ("fused_gate_up", C.c_int),
                ("gate_up", _QW), ("proj", _QW), ("gate_layer", _QW), ("down", _QW),
                ("norm_q", C.c_void_p), ("norm_k", C.c_void_p)]


class _Cfg(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("heads", C.c_int64), ("head_dim", C.c_int64), ("mlp", C.c_int64)]


def _block_args(cfg, weights, x, mod, prefix_k, prefix_v, mask, keep):
    x = _c(x, np.float32)
    b, s, hid = x.shape

    def qw(name):
        if name not in weights:
            return _QW(0, None, 0, 0)
        t, data, rows, cols = weights[name]
        arr = _c(data, np.uint8)
        keep.append(arr)
        return _QW(t, arr.ctypes.data, rows, cols)

    nq, nk = _c(weights["norm_q"], np.float32), _c(weights["norm_k"], np.float32)
    keep += [nq, nk]
    fused = "gate_up" in weights
    bw = _BW(qw("to_q"), qw("to_k"), qw("to_v"), qw("to_out"), 1 if fused else 0, qw("gate_up"), qw("proj"),
             qw("gate_layer"), qw("down"), nq.ctypes.data, nk.ctypes.data)
    c = _Cfg(cfg["hidden"], cfg["heads"], cfg["head_dim"], cfg["mlp"])
    p = 0
    pk = pv = None
    if prefix_k is not None:
        pk, pv = _c(prefix_k, np.uint16), _c(prefix_v, np.uint16)
        p = pk.shape[2]
    mk, mstride = None, 0
    if mask is not None:
        mk = _c(mask, np.uint8)
        mstride = 0 if mk.shape[0] == 1 else s * (p + s)
    mod = _c(mod, np.float32)
    keep += [x, mod, pk, pv, mk]
    return x, b, s, bw, c, mod, pk, pv, p, mk, mstride


def block_forward(cfg, weights, x, mod, pe, prefix_k=None, prefix_v=None, mask=None, mode=CANDLE):
    """TransformerBlock::forward. cfg: dict(hidden, heads, head_dim, mlp). weights: dict name ->
    (type, bytes, rows, cols) for to_q, to_k, to_v, to_out, gate_up | (proj, gate_layer), down;
    plus norm_q / norm_k f32 arrays. x [B,S,h]; mod [B, 1|S, 4h]; pe [S, D];
    prefix_k/v bf16 (uint16) [B,H,P,D]. Returns (x_out, k [B,H,S,D], v [B,H,S,D])."""
    keep = []
    x, b, s, bw, c, mod, pk, pv, p, mk, mstride = _block_args(cfg, weights, x, mod, prefix_k, prefix_v, mask, keep)
    H, D = cfg["heads"], cfg["head_dim"]
    xo = np.empty_like(x)
    ko = np.empty((b, H, s, D), dtype=np.float32)
    vo = np.empty((b, H, s, D), dtype=np.float32)
    pe = _c(pe, np.float32)
    rc = lib().oq_block_forward(C.byref(c), C.byref(bw), _p(x), b, s, _p(mod), mod.shape[1],
                                _p(pe), _p(mk), mstride, _p(pk), _p(pv), p, _p(xo), _p(ko),
                                _p(vo), mode)
    if rc != 0:
        raise ValueError(f"oq_block_forward -> {rc}")
    return xo, ko, vo


def block_forward_rows(cfg, weights, x, mod, pe, rows, prefix_k=None, prefix_v=None, mask=None, mode=CANDLE):
    """block_forward for the token rows `rows` (flat indices b*S + t): returns (x_out [len(rows), h],
    k [B,H,S,D], v [B,H,S,D]); each row equals that row of block_forward bit for bit."""
    keep = []
    x, b, s, bw, c, mod, pk, pv, p, mk, mstride = _block_args(cfg, weights, x, mod, prefix_k, prefix_v, mask, keep)
    H, D = cfg["heads"], cfg["head_dim"]
    r = _c(rows, np.int64)
    xo = np.empty((r.size, x.shape[2]), dtype=np.float32)
    ko = np.empty((b, H, s, D), dtype=np.float32)
    vo = np.empty((b, H, s, D), dtype=np.float32)
    pe = _c(pe, np.float32)
    rc = lib().oq_block_forward_rows(C.byref(c), C.byref(bw), _p(x), b, s, _p(mod), mod.shape[1],
                                     _p(pe), _p(mk), mstride, _p(pk), _p(pv), p, _p(r), r.size,
                                     _p(xo), _p(ko), _p(vo), mode)
    if rc != 0:
        raise ValueError(f"oq_block_forward_rows -> {rc}")
    return xo, ko, vo


def timestep_embedding(t, dim=256):
    t = _c(np.atleast_1d(t), np.float32)
    out = np.empty((t.size, dim), dtype=np.float32)
    lib().oq_timestep_embedding(_p(t), t.size, dim, _p(out))
    return out


def now():
    return float(lib().oq_now_seconds())


def num_threads():
    return int(lib().oq_num_threads())
