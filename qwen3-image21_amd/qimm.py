"""ctypes binding of libqimm.so, the C ABI declared in include/qimm.h.

Thin host-side mirror of the reference's block interface for Python callers
(tests, benchmark): device buffers are passed as integer device addresses
(e.g. ``torch.Tensor.data_ptr()``) and streams as ``hipStream_t`` handles
(e.g. ``torch.cuda.current_stream().cuda_stream``).

Loading order matters on ROCm: import torch first when torch is used, so this
library binds to the HIP runtime torch already loaded (same SONAME) and
torch's streams and allocations are valid here.

The library is required: loading fails loudly when libqimm.so is missing; there
is no fallback implementation.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libqimm.so")

# GGML type ids (include/qimm.h)
F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30

OK = 0
STATUS = {0: "QIMM_OK", 1: "QIMM_ERR_ARG", 2: "QIMM_ERR_SHAPE", 3: "QIMM_ERR_TYPE",
          4: "QIMM_ERR_OOM", 5: "QIMM_ERR_HIP", 6: "QIMM_ERR_STATE", 7: "QIMM_ERR_NOT_FOUND",
          8: "QIMM_ERR_FORMAT"}

# Every symbol include/qimm.h declares: (name, restype, argtypes)
_vp, _i64, _i32, _f32 = C.c_void_p, C.c_int64, C.c_int, C.c_float
SIGNATURES = [
    ("qimm_abi_version", _i32, []),
    ("qimm_status_string", C.c_char_p, [_i32]),
    ("qimm_ctx_create", _i32, [_i32, C.POINTER(_vp)]),
    ("qimm_ctx_destroy", _i32, [_vp]),
    ("qimm_last_error", C.c_char_p, [_vp]),
    ("qimm_malloc", _i32, [_vp, C.c_size_t, C.POINTER(_vp)]),
    ("qimm_free", _i32, [_vp, _vp]),
    ("qimm_memcpy_h2d", _i32, [_vp, _vp, _vp, C.c_size_t, _vp]),
    ("qimm_memcpy_d2h", _i32, [_vp, _vp, _vp, C.c_size_t, _vp]),
    ("qimm_stream_synchronize", _i32, [_vp, _vp]),
    ("qimm_weight_upload", _i32, [_vp, _i32, _i64, _i64, _vp, C.c_size_t, C.POINTER(_vp)]),
    ("qimm_weight_free", _i32, [_vp]),
    ("qimm_weight_device_bytes", _i64, [_vp]),
    ("qimm_dequant", _i32, [_vp, _i32, _vp, _i64, _vp, _vp]),
    ("qimm_qmatmul", _i32, [_vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    ("qimm_qmatmul_noalloc", _i32, [_vp, _vp, _vp, _i64, _i64, _vp, _i32, _vp]),
    ("qimm_qmatmul_scratch_bytes", _i64, [_vp, _i64]),
    ("qimm_joint_layout", _i32, [_i64, _vp, _vp, _i64, _i64, _i64, _vp, _i64,
                                 C.POINTER(_i64), C.POINTER(_i64), C.POINTER(_i64)]),
    ("qimm_rope_table", _i32, [_vp, _i64, _vp, _i64, _vp, C.c_double, _vp]),
    ("qimm_kv_create", _i32, [_vp, _i64, _i64, _i64, _i64, _i64, C.POINTER(_vp)]),
    ("qimm_kv_destroy", _i32, [_vp]),
    ("qimm_kv_store_layer", _i32, [_vp, _i64, _vp, _vp, _vp]),
    ("qimm_kv_load_layer", _i32, [_vp, _i64, _vp, _vp, _vp]),
    ("qimm_kv_prefix_len", _i64, [_vp]),
    ("qimm_kv_create_host", _i32, [_vp, _i64, _i64, _i64, _i64, _i64, C.POINTER(_vp)]),
    ("qimm_kv_is_host", _i32, [_vp]),
    ("qimm_kv_prefetch", _i32, [_vp, _i64, _vp]),
    ("qimm_qk_norm_rope", _i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    ("qimm_v_transpose", _i32, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    ("qimm_attention", _i32, [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _f32, _vp, _vp]),
    ("qimm_attention_masked", _i32, [_vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _vp, _i64, _f32, _vp, _vp, _vp]),
    ("qimm_block_create", _i32, [_vp, _vp, _vp, C.POINTER(_vp)]),
    ("qimm_block_destroy", _i32, [_vp]),
    ("qimm_block_forward", _i32, [_vp, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    ("qimm_block_reserve", _i32, [_vp, _i64, _i64, _i64]),
    ("qimm_block_set_act_mode", _i32, [_vp, _i32]),
    ("qimm_block_act_mode", _i32, [_vp]),
    ("qimm_quantize_act", _i32, [_vp, _i32, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    ("qimm_block_forward_masked", _i32, [_vp, _vp, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp,
                                         _vp]),
    ("qimm_block_profile", _i32, [_vp, _i32]),
    ("qimm_block_stage_times", _i32, [_vp, C.POINTER(C.c_float), _i32]),
    ("qimm_model_create", _i32, [_vp, _vp, _vp, _vp, C.POINTER(_vp)]),
    ("qimm_model_destroy", _i32, [_vp]),
    ("qimm_timestep_embedding", _i32, [_vp, _vp, _i64, _vp, _vp]),
    ("qimm_model_forward", _i32, [_vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp]),
    ("qimm_model_prefix_fill", _i32, [_vp, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _vp]),
    ("qimm_joint_layout_pieces", _i32, [_i64, _vp, _vp, _i64, _vp, _i64, C.POINTER(_i64)]),
    ("qimm_flow_match_sigmas", _i32, [_i64, _i64, _vp]),
    ("qimm_euler_step", _i32, [_vp, _vp, _vp, _i64, _f32, _vp]),
    ("qimm_cfg_combine", _i32, [_vp, _vp, _vp, _i64, _f32, _vp, _vp]),
    ("qimm_gguf_open", _i32, [C.c_char_p, C.POINTER(_vp), C.c_char_p, C.c_size_t]),
    ("qimm_gguf_close", _i32, [_vp]),
    ("qimm_gguf_header", _i32, [_vp, C.POINTER(C.c_uint32), C.POINTER(_i64), C.POINTER(_i64),
                                C.POINTER(C.c_uint32), C.POINTER(C.c_uint64)]),
    ("qimm_gguf_tensor_at", _i32, [_vp, _i64, _vp]),
    ("qimm_gguf_find", _i32, [_vp, C.c_char_p, _vp]),
    ("qimm_gguf_meta_at", _i32, [_vp, _i64, C.POINTER(C.c_char_p), C.POINTER(_i32), C.POINTER(_i32),
                                 C.POINTER(C.c_uint64)]),
    ("qimm_gguf_meta_int", _i32, [_vp, C.c_char_p, C.POINTER(_i64)]),
    ("qimm_gguf_meta_float", _i32, [_vp, C.c_char_p, C.POINTER(C.c_double)]),
    ("qimm_gguf_meta_string", _i32, [_vp, C.c_char_p, C.POINTER(_vp), C.POINTER(C.c_uint64)]),
    ("qimm_gguf_is_known_name", _i32, [C.c_char_p]),
    ("qimm_gguf_block_tensors", _i32, [_vp, _i64, _vp, C.c_char_p, C.c_size_t]),
    ("qimm_gguf_model_tensors", _i32, [_vp, _vp, C.c_char_p, C.c_size_t]),
]
BLOCK_STAGES = ("norm1", "qkv", "attention", "attn_round", "out_proj", "norm2", "gate_up", "hidden_round", "down")
# activation arithmetic at the block's quantized matmul inputs (qimm_block_set_act_mode)
ACT_CANDLE, ACT_BF16 = 0, 1


class BlockConfig(C.Structure):
    _fields_ = [("hidden", _i64), ("heads", _i64), ("head_dim", _i64), ("mlp", _i64)]


class Tensor(C.Structure):
    """qimm_tensor: one GGUF tensor in host memory."""
    _fields_ = [("ggml_type", _i32), ("rows", _i64), ("cols", _i64), ("data", _vp),
                ("nbytes", C.c_size_t)]


class BlockTensors(C.Structure):
    _fields_ = [(n, Tensor) for n in ("to_q", "to_k", "to_v", "to_out", "norm_q", "norm_k",
                                      "gate_up", "proj", "gate_layer", "mlp_out")]


class ModelConfig(C.Structure):
    _fields_ = [("in_channels", _i64), ("joint_dim", _i64), ("hidden", _i64), ("layers", _i64)]


class ModelTensors(C.Structure):
    _fields_ = [(n, Tensor) for n in ("img_in", "t_linear_1", "t_linear_2", "modulation", "norm_out", "proj_out",
                                      "txt_norm", "txt_in", "txt_out")]


class AttnMask(C.Structure):
    """qimm_attn_mask: image_ids int32 [seq] (-1 = text), key_valid uint8 [batch][keys]."""
    _fields_ = [("image_ids", _vp), ("key_valid", _vp)]


class GgufTensorInfo(C.Structure):
    """qimm_gguf_tensor_info."""
    _fields_ = [("name", C.c_char_p), ("ggml_type", _i32), ("n_dims", C.c_int32), ("ne", _i64 * 4),
                ("data", _vp), ("nbytes", C.c_size_t), ("offset", C.c_uint64)]


class QimmError(RuntimeError):
    def __init__(self, msg, status=None):
        super().__init__(msg)
        self.status = status


_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libqimm.so once; raise if it is missing (no fallback path)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise QimmError(f"libqimm.so not built at {path}; run __graft_entry__.build()")
    try:  # bind to the HIP runtime torch ships (same SONAME) rather than a second copy
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(path)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def status_name(rc: int) -> str:
    return STATUS.get(rc, f"status {rc}")


class Context:
    """One device context (qimm_ctx)."""

    def __init__(self, device: int = 0):
        self.lib = load()
        h = C.c_void_p()
        rc = self.lib.qimm_ctx_create(device, C.byref(h))
        if rc != OK:
            raise QimmError(f"qimm_ctx_create({device}) -> {status_name(rc)}")
        self.h = h

    def check(self, rc: int, what: str):
        if rc != OK:
            msg = self.lib.qimm_last_error(self.h)
            raise QimmError(f"{what} -> {status_name(rc)}: {msg.decode() if msg else ''}")

    def close(self):
        if getattr(self, "h", None):
            self.lib.qimm_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- weights --
    def upload(self, ggml_type: int, rows: int, cols: int, data: bytes) -> "Weight":
        h = C.c_void_p()
        buf = C.create_string_buffer(bytes(data), len(data))
        self.check(self.lib.qimm_weight_upload(self.h, ggml_type, rows, cols, buf, len(data), C.byref(h)),
                   "qimm_weight_upload")
        return Weight(self, h, ggml_type, rows, cols)

    def dequant(self, ggml_type: int, dev_bytes: int, n: int, dev_out: int, stream: int = 0):
        self.check(self.lib.qimm_dequant(self.h, ggml_type, dev_bytes, n, dev_out, stream), "qimm_dequant")

    def qmatmul(self, w: "Weight", x_dev: int, m: int, lda: int, y_dev: int, out_type: int, stream: int = 0):
        self.check(self.lib.qimm_qmatmul(self.h, w.h, x_dev, m, lda, y_dev, out_type, stream), "qimm_qmatmul")

    def qmatmul_noalloc(self, w: "Weight", x_dev: int, m: int, lda: int, y_dev: int, out_type: int, stream: int = 0):
        """qmatmul with the library's static per-device scratch: no device allocation in the call."""
        self.check(self.lib.qimm_qmatmul_noalloc(self.h, w.h, x_dev, m, lda, y_dev, out_type, stream),
                   "qimm_qmatmul_noalloc")

    def quantize_act(self, weight_type: int, x_dev: int, m: int, k: int, out_dev: int, ldx: int | None = None,
                     ldo: int | None = None, stream: int = 0):
        """candle's activation rounding of f32 rows x [m, k] to the bf16 operands of a matmul with a
        weight of weight_type (qimm_quantize_act)."""
        self.check(self.lib.qimm_quantize_act(self.h, weight_type, x_dev, m, k, ldx or k, out_dev, ldo or k, stream),
                   "qimm_quantize_act")

    def qmatmul_scratch_bytes(self, w: "Weight", m: int) -> int:
        """Device scratch bytes of the product of w with m rows (qimm_qmatmul_scratch_bytes)."""
        return int(self.lib.qimm_qmatmul_scratch_bytes(w.h, m))

    # -- cache --
    def kv_create(self, layers: int, batch: int, heads: int, prefix_len: int, head_dim: int = 128) -> "KvCache":
        h = C.c_void_p()
        self.check(self.lib.qimm_kv_create(self.h, layers, batch, heads, prefix_len, head_dim, C.byref(h)),
                   "qimm_kv_create")
        return KvCache(self, h, layers, batch, heads, prefix_len)

    # -- the denoising step around the blocks --
    def model_create(self, cfg: ModelConfig, tensors: ModelTensors, blocks) -> "Model":
        arr = (C.c_void_p * max(1, len(blocks)))(*[b.h for b in blocks])
        h = C.c_void_p()
        self.check(self.lib.qimm_model_create(self.h, C.byref(cfg), C.byref(tensors), arr, C.byref(h)),
                   "qimm_model_create")
        return Model(self, h, list(blocks))

    def timestep_embedding(self, t, out_dev, stream=0):
        """t: sequence of floats (one per batch row) -> out_dev f32 [len(t), 256]."""
        arr = (C.c_float * len(t))(*t)
        self.check(self.lib.qimm_timestep_embedding(self.h, arr, len(t), out_dev, stream), "qimm_timestep_embedding")

    def euler_step(self, latents_dev, pred_dev, n, dt, stream=0):
        self.check(self.lib.qimm_euler_step(self.h, latents_dev, pred_dev, n, dt, stream), "qimm_euler_step")

    def cfg_combine(self, cond_dev, neg_dev, n, scale, out_dev, stream=0):
        self.check(self.lib.qimm_cfg_combine(self.h, cond_dev, neg_dev, n, scale, out_dev, stream),
                   "qimm_cfg_combine")

    def kv_create_host(self, layers: int, batch: int, heads: int, prefix_len: int,
                       head_dim: int = 128) -> "KvCache":
        """The host-resident cache (pinned host memory, two device staging slots)."""
        h = C.c_void_p()
        self.check(self.lib.qimm_kv_create_host(self.h, layers, batch, heads, prefix_len, head_dim, C.byref(h)),
                   "qimm_kv_create_host")
        return KvCache(self, h, layers, batch, heads, prefix_len)

    # -- attention --
    def qk_norm_rope(self, x_dev, batch, seq, heads, norm_w_dev, pe_dev, out_dev, stream=0):
        self.check(self.lib.qimm_qk_norm_rope(self.h, x_dev, batch, seq, heads, norm_w_dev, pe_dev, out_dev,
                                              stream), "qimm_qk_norm_rope")

    def v_transpose(self, x_dev, batch, seq, heads, vt_dev, stream=0):
        self.check(self.lib.qimm_v_transpose(self.h, x_dev, batch, seq, heads, vt_dev, stream), "qimm_v_transpose")

    def attention(self, q_dev, batch, heads, sq, kv, layer, k_own, vt_own, so, scale, out_dev, stream=0):
        self.check(self.lib.qimm_attention(self.h, q_dev, batch, heads, sq, kv.h if kv else None, layer,
                                           k_own, vt_own, so, scale, out_dev, stream), "qimm_attention")

    def attention_masked(self, q_dev, batch, heads, sq, kv, layer, k_own, vt_own, so, scale, out_dev,
                         image_ids=None, key_valid=None, stream=0):
        m = AttnMask(image_ids, key_valid)
        self.check(self.lib.qimm_attention_masked(self.h, q_dev, batch, heads, sq, kv.h if kv else None, layer,
                                                  k_own, vt_own, so, scale, C.byref(m), out_dev, stream),
                   "qimm_attention_masked")

    # -- block --
    def block_create(self, cfg: BlockConfig, tensors: BlockTensors) -> "Block":
        h = C.c_void_p()
        self.check(self.lib.qimm_block_create(self.h, C.byref(cfg), C.byref(tensors), C.byref(h)),
                   "qimm_block_create")
        return Block(self, h, cfg)


class Weight:
    def __init__(self, ctx, h, t, rows, cols):
        self.ctx, self.h, self.ggml_type, self.rows, self.cols = ctx, h, t, rows, cols

    def device_bytes(self) -> int:
        return int(self.ctx.lib.qimm_weight_device_bytes(self.h))

    def free(self):
        if self.h:
            self.ctx.lib.qimm_weight_free(self.h)
            self.h = None


class KvCache:
    def __init__(self, ctx, h, layers, batch, heads, prefix_len):
        self.ctx, self.h = ctx, h
        self.layers, self.batch, self.heads, self.prefix_len = layers, batch, heads, prefix_len

    def store(self, layer, k_dev, v_dev, stream=0):
        self.ctx.check(self.ctx.lib.qimm_kv_store_layer(self.h, layer, k_dev, v_dev, stream), "qimm_kv_store_layer")

    def load(self, layer, k_dev, v_dev, stream=0):
        self.ctx.check(self.ctx.lib.qimm_kv_load_layer(self.h, layer, k_dev, v_dev, stream), "qimm_kv_load_layer")

    def prefetch(self, layer, stream=0):
        self.ctx.check(self.ctx.lib.qimm_kv_prefetch(self.h, layer, stream), "qimm_kv_prefetch")

    @property
    def is_host(self) -> bool:
        return bool(self.ctx.lib.qimm_kv_is_host(self.h))

    def free(self):
        if self.h:
            self.ctx.lib.qimm_kv_destroy(self.h)
            self.h = None


class Block:
    def __init__(self, ctx, h, cfg):
        self.ctx, self.h, self.cfg = ctx, h, cfg

    def reserve(self, batch, seq, mod_rows=1):
        """Pre-size the context scratch so forwards up to batch x seq tokens do not allocate."""
        self.ctx.check(self.ctx.lib.qimm_block_reserve(self.h, batch, seq, mod_rows), "qimm_block_reserve")

    def set_act_mode(self, mode: int):
        """ACT_CANDLE (default): the reference CPU path's int8 activation rounding; ACT_BF16: bf16 operands."""
        self.ctx.check(self.ctx.lib.qimm_block_set_act_mode(self.h, mode), "qimm_block_set_act_mode")

    @property
    def act_mode(self) -> int:
        return self.ctx.lib.qimm_block_act_mode(self.h)

    def forward(self, x_dev, x_out_dev, batch, seq, mod_dev, pe_dev, kv=None, layer=0, k_out=None, v_out=None,
                stream=0):
        self.ctx.check(self.ctx.lib.qimm_block_forward(self.h, x_dev, x_out_dev, batch, seq, mod_dev, pe_dev,
                                                       kv.h if kv else None, layer, k_out, v_out, stream),
                       "qimm_block_forward")

    def forward_masked(self, x_dev, x_out_dev, batch, seq, mod_dev, mod_rows, pe_dev, image_ids=None,
                       key_valid=None, kv=None, layer=0, k_out=None, v_out=None, stream=0):
        """Prefix pass: per-token modulation rows (mod_rows 1 or seq) and the block-causal / key mask."""
        m = AttnMask(image_ids, key_valid)
        self.ctx.check(self.ctx.lib.qimm_block_forward_masked(self.h, x_dev, x_out_dev, batch, seq, mod_dev,
                                                              mod_rows, pe_dev, C.byref(m), kv.h if kv else None,
                                                              layer, k_out, v_out, stream),
                       "qimm_block_forward_masked")

    def profile(self, enable: bool = True):
        self.ctx.check(self.ctx.lib.qimm_block_profile(self.h, 1 if enable else 0), "qimm_block_profile")

    def stage_times(self) -> dict:
        """ms per stage of the last forward since profiling was enabled."""
        ms = (C.c_float * len(BLOCK_STAGES))()
        self.ctx.check(self.ctx.lib.qimm_block_stage_times(self.h, ms, len(BLOCK_STAGES)), "qimm_block_stage_times")
        return dict(zip(BLOCK_STAGES, list(ms)))

    def free(self):
        if self.h:
            self.ctx.lib.qimm_block_destroy(self.h)
            self.h = None


def make_tensor(ggml_type: int, rows: int, cols: int, data: bytes | None, keep: list) -> Tensor:
    """qimm_tensor over host bytes; `keep` holds the buffer alive."""
    if data is None:
        return Tensor(0, 0, 0, None, 0)
    buf = C.create_string_buffer(bytes(data), len(data))
    keep.append(buf)
    return Tensor(ggml_type, rows, cols, C.cast(buf, C.c_void_p), len(data))


def joint_layout(text_len: int, text_image_mask=None, cond_shapes=(), target=(1, 1)):
    """JointLayout::new restated host-side: returns (image_ids, prefix_len, target_len)."""
    lib = load()
    cap = text_len * 8 + sum(h * w for h, w in cond_shapes) + target[0] * target[1] + 16
    ids = (C.c_int64 * cap)()
    mask = None
    if text_image_mask is not None:
        mask = (C.c_uint8 * max(1, text_len))(*[1 if m else 0 for m in text_image_mask])
    flat = [v for hw in cond_shapes for v in hw]
    shapes = (C.c_int64 * max(1, len(flat)))(*flat)
    pl, tl, total = C.c_int64(), C.c_int64(), C.c_int64()
    rc = lib.qimm_joint_layout(text_len, mask, shapes, len(cond_shapes), target[0], target[1], ids, cap,
                               C.byref(pl), C.byref(tl), C.byref(total))
    if rc != OK:
        raise QimmError(f"qimm_joint_layout -> {status_name(rc)}")
    return list(ids[: total.value]), pl.value, tl.value


def rope_table(shapes, image_mask, axes=(16, 56, 56), theta=10000.0):
    """EmbedNd::forward restated host-side: returns pe [seq, sum(axes)] f32."""
    import numpy as np
    lib = load()
    seq = len(image_mask)
    width = int(sum(axes))
    pe = np.zeros((seq, width), dtype=np.float32)
    flat = np.array([v for s in shapes for v in s], dtype=np.int64)
    m = np.array([1 if v else 0 for v in image_mask], dtype=np.uint8)
    ax = np.array(axes, dtype=np.int64)
    rc = lib.qimm_rope_table(flat.ctypes.data if len(flat) else None, len(shapes),
                             m.ctypes.data if seq else None, seq, ax.ctypes.data, theta,
                             pe.ctypes.data if seq else None)
    if rc != OK:
        raise QimmError(f"qimm_rope_table -> {status_name(rc)}")
    return pe


class GGUF:
    """A GGUF v2/v3 file opened through the library's reader (qimm_gguf_*):
    memory-mapped, validated at open, tensor data exposed as host pointers."""

    def __init__(self, path: str):
        self.lib = load()
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = self.lib.qimm_gguf_open(path.encode(), C.byref(h), err, len(err))
        if rc != OK:
            raise QimmError(f"qimm_gguf_open({path}) -> {status_name(rc)}: {err.value.decode()}", rc)
        self.h = h

    def close(self):
        if getattr(self, "h", None):
            self.lib.qimm_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def header(self) -> dict:
        v, a = C.c_uint32(), C.c_uint32()
        nt, nkv, off = C.c_int64(), C.c_int64(), C.c_uint64()
        self._ok(self.lib.qimm_gguf_header(self.h, C.byref(v), C.byref(nt), C.byref(nkv), C.byref(a), C.byref(off)),
                 "qimm_gguf_header")
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nkv.value, "alignment": a.value,
                "data_offset": off.value}

    @staticmethod
    def _info(ti: GgufTensorInfo) -> dict:
        raw = C.string_at(ti.data, ti.nbytes) if ti.data else None
        return {"name": ti.name.decode(), "ggml_type": ti.ggml_type, "ne": tuple(ti.ne[:ti.n_dims]),
                "offset": ti.offset, "nbytes": ti.nbytes, "data": raw, "ptr": ti.data}

    def tensors(self) -> list:
        out = []
        for i in range(self.header()["n_tensors"]):
            ti = GgufTensorInfo()
            self._ok(self.lib.qimm_gguf_tensor_at(self.h, i, C.byref(ti)), "qimm_gguf_tensor_at")
            out.append(self._info(ti))
        return out

    def find(self, name: str):
        ti = GgufTensorInfo()
        rc = self.lib.qimm_gguf_find(self.h, name.encode(), C.byref(ti))
        if rc == 7:
            return None
        self._ok(rc, f"qimm_gguf_find({name})")
        return self._info(ti)

    def metadata(self) -> list:
        """[(key, value_type, element_type, count)] in file order."""
        out = []
        for i in range(self.header()["n_kv"]):
            k, t, et, n = C.c_char_p(), C.c_int(), C.c_int(), C.c_uint64()
            self._ok(self.lib.qimm_gguf_meta_at(self.h, i, C.byref(k), C.byref(t), C.byref(et), C.byref(n)),
                     "qimm_gguf_meta_at")
            out.append((k.value.decode(), t.value, et.value, n.value))
        return out

    def meta_int(self, key: str) -> int:
        v = C.c_int64()
        self._ok(self.lib.qimm_gguf_meta_int(self.h, key.encode(), C.byref(v)), f"qimm_gguf_meta_int({key})")
        return v.value

    def meta_float(self, key: str) -> float:
        v = C.c_double()
        self._ok(self.lib.qimm_gguf_meta_float(self.h, key.encode(), C.byref(v)), f"qimm_gguf_meta_float({key})")
        return v.value

    def meta_string(self, key: str) -> str:
        p, n = C.c_void_p(), C.c_uint64()
        self._ok(self.lib.qimm_gguf_meta_string(self.h, key.encode(), C.byref(p), C.byref(n)),
                 f"qimm_gguf_meta_string({key})")
        return C.string_at(p, n.value).decode()

    def model_tensors(self) -> ModelTensors:
        """The global tensors for Context.model_create (pointers valid while open)."""
        T = ModelTensors()
        err = C.create_string_buffer(512)
        rc = self.lib.qimm_gguf_model_tensors(self.h, C.byref(T), err, len(err))
        self._ok(rc, "qimm_gguf_model_tensors", err.value.decode())
        return T

    def block_tensors(self, layer: int) -> BlockTensors:
        """transformer_blocks.{layer} for Context.block_create; pointers stay
        valid while this file is open."""
        T = BlockTensors()
        err = C.create_string_buffer(512)
        rc = self.lib.qimm_gguf_block_tensors(self.h, layer, C.byref(T), err, len(err))
        self._ok(rc, f"qimm_gguf_block_tensors({layer})", err.value.decode())
        return T

    def _ok(self, rc, what, detail=""):
        if rc != OK:
            raise QimmError(f"{what} -> {status_name(rc)} {detail}".rstrip(), rc)


def gguf_is_known_name(name: str) -> bool:
    return bool(load().qimm_gguf_is_known_name(name.encode()))


class Model:
    """The transformer around the blocks (qimm_model)."""

    def __init__(self, ctx, h, blocks):
        self.ctx, self.h, self.blocks = ctx, h, blocks  # blocks kept alive: the model does not own them

    def forward(self, latents_dev, batch, seq, t_sin_dev, pe_dev, kv, pred_dev, key_valid_dev=None, stream=0):
        self.ctx.check(self.ctx.lib.qimm_model_forward(self.h, latents_dev, batch, seq, t_sin_dev, pe_dev,
                                                       kv.h if kv else None, key_valid_dev, pred_dev, stream),
                       "qimm_model_forward")

    def prefix_fill(self, txt_dev, text_len, cond_dev, cond_len, batch, pieces, image_ids_dev, key_valid_dev, pe_dev,
                    kv, stream=0):
        flat = [v for p in pieces for v in p]
        arr = (C.c_int64 * max(1, len(flat)))(*flat)
        self.ctx.check(self.ctx.lib.qimm_model_prefix_fill(self.h, txt_dev, text_len, cond_dev, cond_len, batch, arr,
                                                           len(pieces), image_ids_dev, key_valid_dev, pe_dev, kv.h,
                                                           stream), "qimm_model_prefix_fill")

    def free(self):
        if self.h:
            self.ctx.lib.qimm_model_destroy(self.h)
            self.h = None


def flow_match_sigmas(steps: int, image_seq_len: int) -> list:
    out = (C.c_float * steps)()
    rc = load().qimm_flow_match_sigmas(steps, image_seq_len, out)
    if rc != OK:
        raise QimmError(f"qimm_flow_match_sigmas -> {status_name(rc)}", rc)
    return list(out)


def joint_layout_pieces(text_len: int, text_image_mask=None, cond_shapes=()) -> list:
    """(kind, start, len) triples of the prefix: 0 = prompt rows, 1 = condition rows."""
    mask = None
    if text_image_mask is not None:
        mask = (C.c_uint8 * text_len)(*[1 if v else 0 for v in text_image_mask])
    flat = [v for hw in cond_shapes for v in hw]
    shp = (C.c_int64 * max(1, len(flat)))(*flat)
    cap = text_len + len(cond_shapes) + 1
    out = (C.c_int64 * (3 * cap))()
    n = C.c_int64()
    rc = load().qimm_joint_layout_pieces(text_len, mask, shp if flat else None, len(cond_shapes), out, cap, C.byref(n))
    if rc != OK:
        raise QimmError(f"qimm_joint_layout_pieces -> {status_name(rc)}", rc)
    return [tuple(out[3 * i:3 * i + 3]) for i in range(n.value)]
