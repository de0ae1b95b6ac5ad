"""Pure-Python restatement of the GGUF v3 file format: a writer and a reader.

TEST INFRASTRUCTURE ONLY: imported by tests/ to build fixture files and to
check the library's reader, never by the product library.

The reference reads GGUF through candle's gguf_file module (candle-core 0.11,
an external crate, not part of the reference tree); its own code only calls
Content::read / Content::tensor (src/gguf_loader.rs:24-36, src/service.rs:246-258)
and maps names (src/gguf_mapping.rs:13-60). This file restates the published
GGUF layout (ggml docs/gguf.md, version 3), which that reader implements:

    u32 magic 0x46554747 ("GGUF" little-endian), u32 version,
    u64 tensor_count, u64 metadata_kv_count,
    metadata: { string key, u32 value_type, value }*,
    tensor infos: { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset }*,
    zero padding to ALIGNMENT (general.alignment, u32, default 32),
    tensor data: tensor i at data_start + offset_i, offsets multiples of ALIGNMENT.
    string = u64 byte length + UTF-8 bytes (no terminator);
    array = u32 element type + u64 count + elements.

Value types: 0 u8, 1 i8, 2 u16, 3 i16, 4 u32, 5 i32, 6 f32, 7 bool, 8 string,
9 array, 10 u64, 11 i64, 12 f64. All integers little-endian.

Parity pinning: tests/test_gguf_cpu.py checks this reader and the library's
reader against a hand-assembled byte string whose every field is written out
in the test, independent of this writer.
"""
from __future__ import annotations

import struct

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}

# (values per block, bytes per block) of the GGML tensor types used here
BLOCK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210), 30: (1, 2)}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        for it in items:
            out += _value(et, it)
        return out
    return struct.pack(_SCALAR[t], v)


def tensor_nbytes(ggml_type: int, ne) -> int:
    blk, nb = BLOCK[ggml_type]
    n = 1
    for d in ne:
        n *= d
    assert ne[0] % blk == 0
    return n // blk * nb


def write(path: str, metadata, tensors, alignment: int = 32, version: int = 3) -> None:
    """metadata: list of (key, value_type, value); for ARRAY the value is
    (element_type, list). tensors: list of (name, ggml_type, ne tuple with ne[0]
    innermost, raw bytes). general.alignment is written when alignment != 32
    unless the caller already listed it."""
    meta = list(metadata)
    if alignment != 32 and not any(k == "general.alignment" for k, _, _ in meta):
        meta.append(("general.alignment", U32, alignment))
    head = struct.pack("<IIQQ", MAGIC, version, len(tensors), len(meta))
    for k, t, v in meta:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for name, gt, ne, data in tensors:
        assert len(data) == tensor_nbytes(gt, ne), name
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, gt, ne, data), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", gt, o)
    pad = (-len(head)) % alignment
    body = bytearray()
    for (name, gt, ne, data), o in zip(tensors, offsets):
        body += b"\0" * (o - len(body))
        body += data
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad + bytes(body))


class Reader:
    """Parses a whole GGUF file held in memory: .version, .metadata
    {key: (type, value)}, .tensors {name: (ggml_type, ne, absolute offset,
    raw bytes or None for unknown types)}, .alignment, .data_offset."""

    def __init__(self, blob: bytes):
        self.b = blob
        self.p = 0
        magic, self.version = self._u("<II")
        if magic != MAGIC or self.version not in (2, 3):
            raise ValueError("not a GGUF v2/v3 file")
        nt, nkv = self._u("<QQ")
        self.metadata = {}
        for _ in range(nkv):
            k = self._s()
            t = self._u("<I")[0]
            self.metadata[k] = (t, self._v(t))
        self.alignment = self.metadata.get("general.alignment", (U32, 32))[1]
        infos = []
        for _ in range(nt):
            name = self._s()
            nd = self._u("<I")[0]
            ne = self._u("<" + "Q" * nd)
            gt, off = self._u("<IQ")
            infos.append((name, gt, ne, off))
        a = self.alignment
        self.data_offset = (self.p + a - 1) // a * a
        self.tensors = {}
        for name, gt, ne, off in infos:
            start = self.data_offset + off
            raw = None
            if gt in BLOCK:
                n = tensor_nbytes(gt, ne)
                if start + n > len(blob):
                    raise ValueError(f"tensor {name} outside the file")
                raw = blob[start:start + n]
            self.tensors[name] = (gt, tuple(ne), start, raw)

    def _u(self, fmt):
        n = struct.calcsize(fmt)
        if self.p + n > len(self.b):
            raise ValueError("truncated")
        v = struct.unpack_from(fmt, self.b, self.p)
        self.p += n
        return v

    def _s(self):
        n = self._u("<Q")[0]
        if self.p + n > len(self.b):
            raise ValueError("truncated string")
        s = self.b[self.p:self.p + n].decode("utf-8")
        self.p += n
        return s

    def _v(self, t):
        if t == STRING:
            return self._s()
        if t == ARRAY:
            et, n = self._u("<IQ")
            return (et, [self._v(et) for _ in range(n)])
        if t not in _SCALAR:
            raise ValueError(f"unknown value type {t}")
        return self._u(_SCALAR[t])[0]


def read(path: str) -> Reader:
    with open(path, "rb") as f:
        return Reader(f.read())


# The model's tensor names (src/gguf_mapping.rs:13-60) plus the fused gate_up
# (src/quantized_transformer.rs:181), with the ComfyUI prefix of
# src/service.rs:250-256 stripped first.
_GLOBAL = {"time_text_embed.timestep_embedder.linear_1.weight", "time_text_embed.timestep_embedder.linear_2.weight",
           "norm_out.linear.weight", "proj_out.weight", "img_in.weight", "txt_in.in_layer.weight",
           "txt_in.out_layer.weight", "txt_in.text_norm.weight", "modulation.1.weight"}
_BLOCK_SUB = {"attn.to_q.weight", "attn.to_k.weight", "attn.to_v.weight", "attn.to_out.0.weight",
              "attn.norm_q.weight", "attn.norm_k.weight", "img_mlp.proj.weight", "img_mlp.gate_layer.weight",
              "img_mlp.out.weight", "img_mlp.gate_up.weight"}
PREFIX = "model.diffusion_model."


def is_known_name(name: str) -> bool:
    if name.startswith(PREFIX):
        name = name[len(PREFIX):]
    if name in _GLOBAL:
        return True
    if not name.startswith("transformer_blocks."):
        return False
    rest = name[len("transformer_blocks."):]
    idx, _, sub = rest.partition(".")
    if idx.startswith("+"):  # Rust's usize parse takes one leading '+'
        idx = idx[1:]
    return idx.isascii() and idx.isdigit() and sub in _BLOCK_SUB
