"""The GGUF reader (qimm_gguf_*, N3) against the GGUF format, on the CPU.

The reference parses GGUF with candle's external gguf_file module
(Content::read / Content::tensor, called from src/service.rs:246-258 and
src/gguf_loader.rs:24-36) and holds no GGUF fixture, so parity is pinned by:
- a file assembled here field by field from the published v3 layout, with the
  expected values written out (catches a reversed ne order, a missing alignment
  pad, u32 counts, a wrong data origin);
- seeded round trips through the oracle's independent writer (oracle/gguf.py),
  read back by both the oracle's reader and the library;
- every truncation of a small file and a set of corrupted fields, which must
  fail with QIMM_ERR_FORMAT, never crash or point outside the file;
- the name-mapping cases of src/gguf_mapping.rs:76-121.
"""
import struct

import numpy as np
import pytest

import gguf as G
import qimm
import synth


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def gstr(s):
    return u64(len(s)) + s.encode()


def hand_file():
    """GGUF v3, 2 metadata entries, 2 tensors, default alignment 32."""
    head = b"GGUF" + u32(3) + u64(2) + u64(2)
    head += gstr("general.architecture") + u32(8) + gstr("qwen_image")
    head += gstr("qwen_image.block_count") + u32(4) + u32(32)
    # tensor 0: img_in.weight, F32, ne = (4, 2) -> 2 rows of 4, offset 0
    head += gstr("img_in.weight") + u32(2) + u64(4) + u64(2) + u32(0) + u64(0)
    # tensor 1: attn.norm_q of block 3, F16, ne = (4,), offset 32 (32 B of tensor 0, aligned)
    head += gstr("transformer_blocks.3.attn.norm_q.weight") + u32(1) + u64(4) + u32(1) + u64(32)
    pad = (-len(head)) % 32
    t0 = struct.pack("<8f", 1.0, 2.0, 3.0, 4.0, -1.0, -2.0, 0.5, 0.25)
    t1 = struct.pack("<4e", 1.0, -2.0, 0.5, 65504.0)
    return head + b"\0" * pad + t0 + t1, len(head) + pad


def test_hand_assembled_file_both_readers(tmp_path):
    blob, data_off = hand_file()
    p = tmp_path / "hand.gguf"
    p.write_bytes(blob)
    # the oracle reader
    r = G.read(str(p))
    assert r.version == 3 and r.alignment == 32 and r.data_offset == data_off
    assert r.metadata["general.architecture"] == (G.STRING, "qwen_image")
    assert r.metadata["qwen_image.block_count"] == (G.U32, 32)
    assert r.tensors["img_in.weight"][:3] == (0, (4, 2), data_off)
    assert r.tensors["transformer_blocks.3.attn.norm_q.weight"][:3] == (1, (4,), data_off + 32)
    # the library
    with qimm.GGUF(str(p)) as g:
        h = g.header()
        assert h == {"version": 3, "n_tensors": 2, "n_kv": 2, "alignment": 32, "data_offset": data_off}
        t = g.tensors()
        assert [x["name"] for x in t] == ["img_in.weight", "transformer_blocks.3.attn.norm_q.weight"]
        assert t[0]["ne"] == (4, 2) and t[0]["ggml_type"] == 0 and t[0]["nbytes"] == 32
        np.testing.assert_array_equal(np.frombuffer(t[0]["data"], np.float32),
                                      [1, 2, 3, 4, -1, -2, 0.5, 0.25])
        assert t[1]["ne"] == (4,) and t[1]["offset"] == data_off + 32 and t[1]["nbytes"] == 8
        np.testing.assert_array_equal(np.frombuffer(t[1]["data"], np.float16), [1, -2, 0.5, 65504])
        assert g.meta_string("general.architecture") == "qwen_image"
        assert g.meta_int("qwen_image.block_count") == 32
        assert g.metadata() == [("general.architecture", 8, -1, 1), ("qwen_image.block_count", 4, -1, 1)]
        with pytest.raises(qimm.QimmError) as e:
            g.meta_int("general.architecture")
        assert e.value.status == 3  # QIMM_ERR_TYPE
        assert g.find("nope") is None


def test_every_truncation_fails_cleanly(tmp_path):
    blob, _ = hand_file()
    p = tmp_path / "t.gguf"
    for n in range(len(blob)):
        p.write_bytes(blob[:n])
        with pytest.raises(qimm.QimmError) as e:
            qimm.GGUF(str(p))
        assert e.value.status == 8, n  # QIMM_ERR_FORMAT
    p.write_bytes(blob)
    qimm.GGUF(str(p)).close()


@pytest.mark.parametrize("what", ["magic", "version", "n_dims", "type", "offset", "align", "kvtype", "count",
                                  "dup"])
def test_corrupted_fields_rejected(tmp_path, what):
    blob, _ = hand_file()
    b = bytearray(blob)
    name0 = gstr("img_in.weight")
    i0 = blob.index(name0) + len(name0)  # tensor 0: n_dims at i0, ne at i0+4, type at i0+20, offset at i0+24
    if what == "magic":
        b[0:4] = b"GGUG"
    elif what == "version":
        b[4:8] = u32(1)
    elif what == "n_dims":
        b[i0:i0 + 4] = u32(5)
    elif what == "type":  # Q4_K with ne0 = 4: not a whole block
        b[i0 + 20:i0 + 24] = u32(12)
    elif what == "offset":  # 8 is not a multiple of the alignment
        b[i0 + 24:i0 + 32] = u64(8)
    elif what == "align":
        b = bytearray(G_blob_with_alignment(48))
    elif what == "kvtype":
        k = gstr("general.architecture")
        j = blob.index(k) + len(k)
        b[j:j + 4] = u32(13)
    elif what == "count":
        b[8:16] = u64(1 << 60)
    elif what == "dup":  # two tensors named img_in.weight
        head = b"GGUF" + u32(3) + u64(2) + u64(0)
        head += gstr("img_in.weight") + u32(1) + u64(4) + u32(0) + u64(0)
        head += gstr("img_in.weight") + u32(1) + u64(4) + u32(0) + u64(32)
        b = bytearray(head + b"\0" * ((-len(head)) % 32) + b"\0" * 48)
    p = tmp_path / "bad.gguf"
    p.write_bytes(bytes(b))
    with pytest.raises(qimm.QimmError) as e:
        qimm.GGUF(str(p))
    assert e.value.status == 8


@pytest.mark.parametrize("ne", [(1 << 40, 1 << 40, 1 << 40, 1 << 40),   # product is 0 modulo 2^128
                                (1 << 35, 1 << 30, 1, 1)])                 # fits 128 bits, not 64
def test_tensor_size_overflow_rejected(tmp_path, ne):
    """Each dimension passes the per-dimension cap, but the byte count
    ne1 ne2 ne3 (ne0 / 32) 34 of a Q8_0 tensor overflows: a wrapped size must
    not slip past the bounds check."""
    head = b"GGUF" + u32(3) + u64(1) + u64(0)
    head += gstr("img_in.weight") + u32(4) + b"".join(u64(v) for v in ne) + u32(8) + u64(0)
    p = tmp_path / "wrap.gguf"
    p.write_bytes(head + b"\0" * ((-len(head)) % 32) + b"\0" * 64)
    with pytest.raises(qimm.QimmError) as e:
        qimm.GGUF(str(p))
    assert e.value.status == 8


def G_blob_with_alignment(al):
    head = b"GGUF" + u32(3) + u64(0) + u64(1) + gstr("general.alignment") + u32(4) + u32(al)
    return head


def test_tensor_past_end_rejected(tmp_path):
    blob, _ = hand_file()
    p = tmp_path / "short.gguf"
    p.write_bytes(blob[:-1])
    with pytest.raises(qimm.QimmError) as e:
        qimm.GGUF(str(p))
    assert e.value.status == 8
    assert not (tmp_path / "missing.gguf").exists()
    with pytest.raises(qimm.QimmError) as e:
        qimm.GGUF(str(tmp_path / "missing.gguf"))
    assert e.value.status == 1


def random_file(path, seed, alignment=32, prefix="", fused=True, layers=2, hidden=256, mlp=512, globals_=False,
                txt_in=False):
    rng = np.random.default_rng(seed)
    meta = [("general.architecture", G.STRING, "qwen_image"),
            ("general.name", G.STRING, "synthetic é"),
            ("u8", G.U8, 200), ("i8", G.I8, -5), ("u16", G.U16, 65000), ("i16", G.I16, -30000),
            ("i32", G.I32, -(1 << 30)), ("f32", G.F32, 1.5), ("b", G.BOOL, True),
            ("u64", G.U64, (1 << 62) + 3), ("i64", G.I64, -(1 << 50)), ("f64", G.F64, -2.25),
            ("arr_i32", G.ARRAY, (G.I32, [1, -2, 3])), ("arr_s", G.ARRAY, (G.STRING, ["a", "bc", ""])),
            ("big", G.U64, (1 << 64) - 1)]
    tensors = []
    for layer in range(layers):
        pre = f"{prefix}transformer_blocks.{layer}."
        for sub, t, rows, cols in (("attn.to_q.weight", synth.Q4_K, hidden, hidden),
                                   ("attn.to_k.weight", synth.Q4_K, hidden, hidden),
                                   ("attn.to_v.weight", synth.Q6_K, hidden, hidden),
                                   ("attn.to_out.0.weight", synth.Q8_0, hidden, hidden),
                                   ("img_mlp.out.weight", synth.Q6_K, hidden, mlp)):
            _, data, r, c = synth.weight(rng, t, rows, cols)
            tensors.append((pre + sub, t, (c, r), data.tobytes()))
        for sub in ("attn.norm_q.weight", "attn.norm_k.weight"):
            tensors.append((pre + sub, 0, (128,), rng.standard_normal(128).astype(np.float32).tobytes()))
        if fused:
            _, data, r, c = synth.weight(rng, synth.Q4_K, 2 * mlp, hidden)
            tensors.append((pre + "img_mlp.gate_up.weight", synth.Q4_K, (c, r), data.tobytes()))
        else:
            for sub in ("img_mlp.proj.weight", "img_mlp.gate_layer.weight"):
                _, data, r, c = synth.weight(rng, synth.Q4_K, mlp, hidden)
                tensors.append((pre + sub, synth.Q4_K, (c, r), data.tobytes()))
    _, data, r, c = synth.weight(rng, synth.BF16, hidden, 64, std=0.2)  # finite bf16 values
    tensors.append((prefix + "img_in.weight", synth.BF16, (c, r), data.tobytes()))
    if globals_:
        # the model's global tensors (src/gguf_mapping.rs:27-37), [out, in] as ne = (in, out)
        for name, t, rows, cols in (("time_text_embed.timestep_embedder.linear_1.weight", synth.Q8_0, hidden, 256),
                                    ("time_text_embed.timestep_embedder.linear_2.weight", synth.Q4_K, hidden, hidden),
                                    ("modulation.1.weight", synth.Q4_K, 4 * hidden, hidden),
                                    ("norm_out.linear.weight", synth.BF16, hidden, hidden),
                                    ("proj_out.weight", synth.Q6_K, 64, hidden)):
            _, data, r, c = synth.weight(rng, t, rows, cols, std=0.05)
            tensors.append((prefix + name, t, (c, r), data.tobytes()))
        if txt_in:
            tensors.append((prefix + "txt_in.text_norm.weight", 0, (128,),
                            (0.1 * rng.standard_normal(128)).astype(np.float32).tobytes()))
            for name, rows, cols in (("txt_in.in_layer.weight", hidden, 128), ("txt_in.out_layer.weight", hidden, hidden)):
                _, data, r, c = synth.weight(rng, synth.F32, rows, cols, std=0.05)
                tensors.append((prefix + name, 0, (c, r), data.tobytes()))
    G.write(str(path), meta, tensors, alignment=alignment)
    return meta, tensors


@pytest.mark.parametrize("seed,alignment,prefix,fused", [(1, 32, "", True), (2, 64, "model.diffusion_model.", False),
                                                         (3, 256, "", False)])
def test_round_trip_against_oracle(tmp_path, seed, alignment, prefix, fused):
    p = tmp_path / "rt.gguf"
    meta, tensors = random_file(p, seed, alignment, prefix, fused)
    r = G.read(str(p))
    assert r.alignment == alignment
    with qimm.GGUF(str(p)) as g:
        h = g.header()
        assert (h["version"], h["n_tensors"], h["alignment"], h["data_offset"]) == (3, len(tensors), alignment,
                                                                                   r.data_offset)
        got = g.tensors()
        assert [x["name"] for x in got] == [t[0] for t in tensors]
        for x, (name, gt, ne, data) in zip(got, tensors):
            assert x["ggml_type"] == gt and x["ne"] == ne and x["data"] == data
            assert x["offset"] == r.tensors[name][2] and x["offset"] % alignment == 0
            assert r.tensors[name][3] == data
        keys = [m[0] for m in g.metadata()]
        assert keys == [m[0] for m in meta] + (["general.alignment"] if alignment != 32 else [])
        for k, t, v in meta:
            if t == G.STRING:
                assert g.meta_string(k) == v
            elif t in (G.F32, G.F64):
                assert g.meta_float(k) == v
            elif t == G.ARRAY:
                et, items = v
                assert [m for m in g.metadata() if m[0] == k][0][2:] == (et, len(items))
            elif k == "big":
                with pytest.raises(qimm.QimmError):
                    g.meta_int(k)
            else:
                assert g.meta_int(k) == int(v)
        # the ComfyUI prefix is found either way
        assert g.find("img_in.weight")["name"] == prefix + "img_in.weight"
        # block tensors: what qimm_block_create needs, pointing at the file's bytes
        T = g.block_tensors(1)
        by = {t[0]: t for t in tensors}
        pre = f"{prefix}transformer_blocks.1."
        for field, sub in (("to_q", "attn.to_q.weight"), ("to_v", "attn.to_v.weight"),
                           ("to_out", "attn.to_out.0.weight"), ("mlp_out", "img_mlp.out.weight")):
            ft = getattr(T, field)
            name, gt, ne, data = by[pre + sub]
            assert (ft.ggml_type, ft.cols, ft.rows, ft.nbytes) == (gt, ne[0], ne[1], len(data))
            assert qimm.C.string_at(ft.data, ft.nbytes) == data
        assert (T.norm_q.rows, T.norm_q.cols) == (1, 128)
        if fused:
            assert T.gate_up.data and not T.proj.data and not T.gate_layer.data
        else:
            assert not T.gate_up.data and T.proj.data and T.gate_layer.data
        with pytest.raises(qimm.QimmError) as e:
            g.block_tensors(2)
        assert e.value.status == 7 and "transformer_blocks.2.attn.to_q.weight" in str(e.value)


@pytest.mark.parametrize("name,known", [
    # src/gguf_mapping.rs:76-95 (test_identity_global)
    ("time_text_embed.timestep_embedder.linear_1.weight", True),
    ("time_text_embed.timestep_embedder.linear_2.weight", True),
    ("norm_out.linear.weight", True), ("proj_out.weight", True), ("img_in.weight", True),
    ("txt_in.in_layer.weight", True), ("txt_in.out_layer.weight", True), ("txt_in.text_norm.weight", True),
    ("modulation.1.weight", True),
    # src/gguf_mapping.rs:97-111 (test_identity_blocks)
    ("transformer_blocks.0.attn.to_q.weight", True), ("transformer_blocks.5.attn.norm_k.weight", True),
    ("transformer_blocks.31.img_mlp.gate_layer.weight", True),
    ("transformer_blocks.7.img_mlp.gate_up.weight", True), ("transformer_blocks.+7.attn.to_k.weight", True),
    ("model.diffusion_model.transformer_blocks.2.attn.to_out.0.weight", True),
    # src/gguf_mapping.rs:113-120 (test_unmappable)
    ("unknown.weight", False), ("transformer_blocks.0.attn.add_q_proj.weight", False),
    ("transformer_blocks.0.txt_norm1.weight", False),
    ("transformer_blocks.x.attn.to_q.weight", False), ("transformer_blocks..attn.to_q.weight", False),
    ("transformer_blocks.+.attn.to_q.weight", False), ("transformer_blocks.0", False),
    ("transformer_blocks.0.attn.to_q.bias", False)])
def test_name_mapping(name, known):
    assert G.is_known_name(name) == known
    assert qimm.gguf_is_known_name(name) == known


@pytest.mark.parametrize("prefix,txt_in", [("", True), ("model.diffusion_model.", False)])
def test_model_tensors(tmp_path, prefix, txt_in):
    p = tmp_path / "g.gguf"
    _, tensors = random_file(p, 9, 32, prefix, True, layers=1, globals_=True, txt_in=txt_in)
    by = {name[len(prefix):]: (gt, ne, data) for name, gt, ne, data in tensors}
    with qimm.GGUF(str(p)) as g:
        T = g.model_tensors()
        for field, name in (("img_in", "img_in.weight"),
                            ("t_linear_1", "time_text_embed.timestep_embedder.linear_1.weight"),
                            ("t_linear_2", "time_text_embed.timestep_embedder.linear_2.weight"),
                            ("modulation", "modulation.1.weight"), ("norm_out", "norm_out.linear.weight"),
                            ("proj_out", "proj_out.weight"), ("txt_norm", "txt_in.text_norm.weight"),
                            ("txt_in", "txt_in.in_layer.weight"), ("txt_out", "txt_in.out_layer.weight")):
            ft = getattr(T, field)
            if name not in by:
                assert not ft.data and field.startswith("txt")
                continue
            gt, ne, data = by[name]
            rows = ne[1] if len(ne) > 1 else 1
            assert (ft.ggml_type, ft.cols, ft.rows, ft.nbytes) == (gt, ne[0], rows, len(data))
            assert qimm.C.string_at(ft.data, ft.nbytes) == data
    # a file without the globals names the first missing one
    q = tmp_path / "blocks_only.gguf"
    random_file(q, 10, layers=1)
    with qimm.GGUF(str(q)) as g:
        with pytest.raises(qimm.QimmError) as e:
            g.model_tensors()
        assert e.value.status == 7 and "time_text_embed.timestep_embedder.linear_1.weight" in str(e.value)
