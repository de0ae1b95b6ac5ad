"""A block loaded from a GGUF file (qimm_gguf_block_tensors -> qimm_block_create)
runs the same computation as the block built from the same tensor bytes
directly, bit for bit, and matches the oracle (TransformerBlock::new from the
quantized VarBuilder, src/quantized_transformer.rs:249-256, 173-188, with the
ComfyUI prefix of src/service.rs:250-256)."""
import numpy as np
import pytest

import oracle as O
import qimm
from gpu_util import cos_sim, dev, host, max_abs_rel, stream
from test_gguf_cpu import random_file

pytestmark = pytest.mark.gpu

CFG = dict(hidden=256, heads=2, head_dim=128, mlp=768)


def forward(torch, qctx, T, x, mod, pe):
    blk = qctx.block_create(qimm.BlockConfig(CFG["hidden"], CFG["heads"], 128, CFG["mlp"]), T)
    b, s, _ = x.shape
    x_d, mod_d, pe_d = dev(torch, x), dev(torch, mod), dev(torch, pe)
    out = torch.empty_like(x_d)
    blk.forward(x_d.data_ptr(), out.data_ptr(), b, s, mod_d.data_ptr(), pe_d.data_ptr(), None, 0, None, None,
                stream(torch))
    y = host(out)
    blk.free()
    return y


@pytest.mark.parametrize("seed,prefix,fused", [(5, "", True), (6, "model.diffusion_model.", False)])
def test_block_from_gguf(torch_cuda, qctx, tmp_path, seed, prefix, fused):
    p = tmp_path / "m.gguf"
    _, tensors = random_file(p, seed, 32, prefix, fused, layers=2, hidden=CFG["hidden"], mlp=CFG["mlp"])
    rng = np.random.default_rng(seed)
    b, s = 1, 64
    x = rng.standard_normal((b, s, CFG["hidden"])).astype(np.float32)
    mod = (rng.standard_normal((b, 1, 4 * CFG["hidden"])) * 0.5).astype(np.float32)
    pe = O.rope_table([(1, 8, 8)], [1] * s)
    with qimm.GGUF(str(p)) as g:
        y_file = forward(torch_cuda, qctx, g.block_tensors(1), x, mod, pe)
    # the same bytes handed over directly
    by = {name: (gt, ne, data) for name, gt, ne, data in tensors}
    pre = f"{prefix}transformer_blocks.1."
    keep, T = [], qimm.BlockTensors()
    w = {}
    for field, sub in (("to_q", "attn.to_q.weight"), ("to_k", "attn.to_k.weight"), ("to_v", "attn.to_v.weight"),
                       ("to_out", "attn.to_out.0.weight"), ("mlp_out", "img_mlp.out.weight"),
                       ("gate_up", "img_mlp.gate_up.weight"), ("proj", "img_mlp.proj.weight"),
                       ("gate_layer", "img_mlp.gate_layer.weight"), ("norm_q", "attn.norm_q.weight"),
                       ("norm_k", "attn.norm_k.weight")):
        if pre + sub not in by:
            continue
        gt, ne, data = by[pre + sub]
        rows, cols = (ne[1], ne[0]) if len(ne) == 2 else (ne[0], 1)
        setattr(T, field, qimm.make_tensor(gt, rows, cols, data, keep))
        if field.startswith("norm"):
            w[field] = np.frombuffer(data, np.float32)
        else:
            w[{"mlp_out": "down"}.get(field, field)] = (gt, np.frombuffer(data, np.uint8), rows, cols)
    y_direct = forward(torch_cuda, qctx, T, x, mod, pe)
    assert np.array_equal(y_file, y_direct)
    ref, _, _ = O.block_forward(CFG, w, x, mod, pe, None, None, mode=O.CANDLE)
    assert cos_sim(y_file, ref) >= 0.9999 and max_abs_rel(y_file, ref) <= 2e-2


def test_model_from_gguf(torch_cuda, qctx, tmp_path):
    """qimm_gguf_model_tensors + qimm_gguf_block_tensors feed qimm_model_create
    (QwenImageTransformerQuantized::new_with_dtype from the quantized VarBuilder,
    src/quantized_transformer.rs:399-427): the forward equals the model built
    from the same bytes directly, and the oracle."""
    import model as OM
    torch = torch_cuda
    p = tmp_path / "full.gguf"
    layers = 2
    _, tensors = random_file(p, 12, 32, "model.diffusion_model.", True, layers=layers, hidden=CFG["hidden"],
                             mlp=CFG["mlp"], globals_=True, txt_in=True)
    rng = np.random.default_rng(12)
    b, s = 1, 32
    latents = rng.standard_normal((b, s, 64)).astype(np.float32)
    pe = O.rope_table([(1, 4, 8)], [1] * s)
    lat_d, pe_d = dev(torch, latents), dev(torch, pe)
    t_sin = torch.empty((b, 256), dtype=torch.float32, device="cuda")
    qctx.timestep_embedding([0.4], t_sin.data_ptr(), stream(torch))

    def run(model_t, block_t):
        blks = [qctx.block_create(qimm.BlockConfig(CFG["hidden"], CFG["heads"], 128, CFG["mlp"]), bt) for bt in block_t]
        m = qctx.model_create(qimm.ModelConfig(64, 128, CFG["hidden"], layers), model_t, blks)
        pred = torch.empty((b, s, 64), dtype=torch.float32, device="cuda")
        m.forward(lat_d.data_ptr(), b, s, t_sin.data_ptr(), pe_d.data_ptr(), None, pred.data_ptr(), None,
                  stream(torch))
        y = host(pred)
        m.free()
        for x in blks:
            x.free()
        return y

    with qimm.GGUF(str(p)) as g:
        y_file = run(g.model_tensors(), [g.block_tensors(i) for i in range(layers)])
    # the same bytes handed over directly, and the oracle's dicts
    pre = "model.diffusion_model."
    by = {name[len(pre):]: (gt, ne, data) for name, gt, ne, data in tensors}
    keep, MT = [], qimm.ModelTensors()
    gdict = {}
    for field, name in (("img_in", "img_in.weight"), ("t_linear_1", "time_text_embed.timestep_embedder.linear_1.weight"),
                        ("t_linear_2", "time_text_embed.timestep_embedder.linear_2.weight"),
                        ("modulation", "modulation.1.weight"), ("norm_out", "norm_out.linear.weight"),
                        ("proj_out", "proj_out.weight"), ("txt_norm", "txt_in.text_norm.weight"),
                        ("txt_in", "txt_in.in_layer.weight"), ("txt_out", "txt_in.out_layer.weight")):
        gt, ne, data = by[name]
        rows, cols = (ne[1], ne[0]) if len(ne) > 1 else (1, ne[0])
        setattr(MT, field, qimm.make_tensor(gt, rows, cols, data, keep))
        gdict[field] = (gt, np.frombuffer(data, np.uint8), rows, cols)
    bts, bdicts = [], []
    for i in range(layers):
        T, w = qimm.BlockTensors(), {}
        for field, sub in (("to_q", "attn.to_q.weight"), ("to_k", "attn.to_k.weight"), ("to_v", "attn.to_v.weight"),
                           ("to_out", "attn.to_out.0.weight"), ("mlp_out", "img_mlp.out.weight"),
                           ("gate_up", "img_mlp.gate_up.weight"), ("norm_q", "attn.norm_q.weight"),
                           ("norm_k", "attn.norm_k.weight")):
            gt, ne, data = by[f"transformer_blocks.{i}.{sub}"]
            rows, cols = (ne[1], ne[0]) if len(ne) > 1 else (ne[0], 1)
            setattr(T, field, qimm.make_tensor(gt, rows, cols, data, keep))
            if field.startswith("norm"):
                w[field] = np.frombuffer(data, np.float32)
            else:
                w[{"mlp_out": "down"}.get(field, field)] = (gt, np.frombuffer(data, np.uint8), rows, cols)
        bts.append(T)
        bdicts.append(w)
    y_direct = run(MT, bts)
    assert np.array_equal(y_file, y_direct)
    ref = OM.model_forward(CFG, gdict, bdicts, latents, O.timestep_embedding(np.array([0.4], np.float32)), pe)
    assert cos_sim(y_file, ref) >= 0.9999 and max_abs_rel(y_file, ref) <= 2e-2
