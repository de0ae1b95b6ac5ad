"""GPU parity of the denoising step around the blocks (N2): the model's cached
forward (forward_conditioned with a filled cache, src/quantized_transformer.rs:471-551),
the prefix fill through txt_in / img_in / zero_modulation / the blocks
(prefix_kv, :359-392), the time embedding (src/scheduler.rs:101-126), the
Euler update and the CFG combine (src/scheduler.rs:54-66, src/pipeline.rs:168-197),
against oracle/model.py on identical seeded inputs. Bars as for the block:
cosine >= 0.9999 and max|a-b|/max|b| <= 2e-2 against the oracle's candle mode
(int8 activations in the blocks), cosine >= 0.9999 against its exact mode; the
f32-only parts (no blocks) to 1e-4 relative."""
import numpy as np
import pytest

import model as OM
import oracle as O
import qimm
import synth
from gpu_util import cos_sim, dev, host, max_abs_rel, stream
from test_gpu_block import SMALL, block_tensors

pytestmark = pytest.mark.gpu

CH, JD = 64, 128


def model_weights(seed, layers):
    rng = np.random.default_rng(seed)
    h = SMALL["hidden"]
    g = {"img_in": synth.weight(rng, synth.F32, h, CH, std=0.2),
         "t_linear_1": synth.weight(rng, synth.Q8_0, h, 256, std=0.05),
         "t_linear_2": synth.weight(rng, synth.Q4_K, h, h, std=0.05),
         "modulation": synth.weight(rng, synth.Q4_K, 4 * h, h, std=0.05),
         "norm_out": synth.weight(rng, synth.BF16, h, h, std=0.05),
         "proj_out": synth.weight(rng, synth.Q6_K, CH, h, std=0.05),
         "txt_norm": synth.weight(rng, synth.F32, 1, JD, std=0.1),
         "txt_in": synth.weight(rng, synth.F32, h, JD, std=0.1),
         "txt_out": synth.weight(rng, synth.Q8_0, h, h, std=0.05)}
    blocks = [synth.block_weights(seed + 100 + i, h, SMALL["heads"], SMALL["mlp"], synth.Q4_K, synth.Q6_K)
              for i in range(layers)]
    return g, blocks


class Built:
    def __init__(self, qctx, g, blocks, joint=JD):
        self.keep = []
        self.blocks = [qctx.block_create(qimm.BlockConfig(SMALL["hidden"], SMALL["heads"], 128, SMALL["mlp"]),
                                         block_tensors(w, self.keep)) for w in blocks]
        T = qimm.ModelTensors()
        for name in ("img_in", "t_linear_1", "t_linear_2", "modulation", "norm_out", "proj_out", "txt_norm",
                     "txt_in", "txt_out"):
            if name in g and joint:
                t, data, rows, cols = g[name]
                setattr(T, name, qimm.make_tensor(t, rows, cols, data.tobytes(), self.keep))
        cfg = qimm.ModelConfig(CH, joint, SMALL["hidden"], len(blocks))
        self.model = qctx.model_create(cfg, T, self.blocks)

    def free(self):
        self.model.free()
        for b in self.blocks:
            b.free()


def t_sin_dev(torch, qctx, ts):
    out = torch.empty((len(ts), 256), dtype=torch.float32, device="cuda")
    qctx.timestep_embedding(list(ts), out.data_ptr(), stream(torch))
    return out


def test_timestep_embedding(torch_cuda, qctx):
    ts = [0.0, 0.02, 0.5, 0.97, 1.0]
    got = host(t_sin_dev(torch_cuda, qctx, ts))
    want = O.timestep_embedding(np.array(ts, np.float32))
    assert np.abs(got - want).max() <= 2e-6
    assert np.array_equal(got[0], OM.zero_sinusoid(1)[0])


def test_euler_and_cfg(torch_cuda, qctx):
    rng = np.random.default_rng(3)
    n = 5000
    x, v, neg = (rng.standard_normal(n).astype(np.float32) for _ in range(3))
    xd, vd, nd = dev(torch_cuda, x), dev(torch_cuda, v), dev(torch_cuda, neg)
    qctx.euler_step(xd.data_ptr(), vd.data_ptr(), n, -0.0625, stream(torch_cuda))
    assert np.allclose(host(xd), x + v * np.float32(-0.0625), rtol=1e-6, atol=1e-7)
    out = torch_cuda.empty_like(vd)
    qctx.cfg_combine(vd.data_ptr(), nd.data_ptr(), n, 4.0, out.data_ptr(), stream(torch_cuda))
    assert np.allclose(host(out), OM.cfg_combine(v, neg, np.float32(4.0)), rtol=1e-6, atol=1e-6)
    qctx.cfg_combine(vd.data_ptr(), nd.data_ptr(), n, 1.0, out.data_ptr(), stream(torch_cuda))
    assert np.allclose(host(out), v, rtol=1e-6, atol=1e-6)


def _target_pe(s_h, s_w, text_len):
    ids, plen, tlen = O.joint_layout(text_len, None, (), (s_h, s_w))
    pe = O.rope_table([(1, s_h, s_w)], [i >= 0 for i in ids])
    return pe, plen


@pytest.mark.parametrize("b,with_kv", [(1, False), (2, True)])
def test_model_forward_cached(torch_cuda, qctx, b, with_kv):
    torch = torch_cuda
    layers, P, sh, sw = 2, 40, 4, 8
    s = sh * sw
    g, blocks = model_weights(11 + b, layers)
    rng = np.random.default_rng(5)
    latents = rng.standard_normal((b, s, CH)).astype(np.float32)
    kc = [O.f32_to_bf16(rng.standard_normal((b, SMALL["heads"], P, 128))) for _ in range(layers)]
    vc = [O.f32_to_bf16(rng.standard_normal((b, SMALL["heads"], P, 128))) for _ in range(layers)]
    pe_full, plen = _target_pe(sh, sw, P)
    pe = pe_full[plen:]
    key_valid = None
    if with_kv:
        key_valid = np.ones((b, P + s), np.uint8)
        key_valid[1, P - 5:P] = 0
    mdl = Built(qctx, g, blocks)
    kv = qctx.kv_create(layers, b, SMALL["heads"], P)
    srcs = []
    for i in range(layers):
        kd, vd = dev(torch, kc[i].view(np.int16)), dev(torch, vc[i].view(np.int16))
        srcs += [kd, vd]
        kv.store(i, kd.data_ptr(), vd.data_ptr(), stream(torch))
    ts = [0.73] * b
    lat_d, pe_d = dev(torch, latents), dev(torch, pe)
    tsd = t_sin_dev(torch, qctx, ts)
    kvd = dev(torch, key_valid) if with_kv else None
    pred = torch.empty((b, s, CH), dtype=torch.float32, device="cuda")
    mdl.model.forward(lat_d.data_ptr(), b, s, tsd.data_ptr(), pe_d.data_ptr(), kv, pred.data_ptr(),
                      kvd.data_ptr() if with_kv else None, stream(torch))
    got = host(pred)
    t_sin = O.timestep_embedding(np.array(ts, np.float32))
    ref = OM.model_forward(SMALL, g, blocks, latents, t_sin, pe, kc, vc, key_valid, mode=O.CANDLE)
    assert cos_sim(got, ref) >= 0.9999 and max_abs_rel(got, ref) <= 2e-2, (cos_sim(got, ref), max_abs_rel(got, ref))
    ref_e = OM.model_forward(SMALL, g, blocks, latents, t_sin, pe, kc, vc, key_valid, mode=O.EXACT)
    assert cos_sim(got, ref_e) >= 0.9999
    kv.free()
    mdl.free()


def test_model_forward_no_blocks_f32_path(torch_cuda, qctx):
    """With no layers the forward is the f32 globals alone: img_in, time
    embedding, norm_out, proj_out (exact f32 weights, f32 accumulation)."""
    torch = torch_cuda
    g, _ = model_weights(21, 0)
    rng = np.random.default_rng(8)
    b, s = 2, 48
    latents = rng.standard_normal((b, s, CH)).astype(np.float32)
    mdl = Built(qctx, g, [])
    tsd = t_sin_dev(torch, qctx, [0.3, 0.9])
    pe = np.zeros((s, 128), np.float32)
    lat_d, pe_d = dev(torch, latents), dev(torch, pe)
    pred = torch.empty((b, s, CH), dtype=torch.float32, device="cuda")
    mdl.model.forward(lat_d.data_ptr(), b, s, tsd.data_ptr(), pe_d.data_ptr(), None, pred.data_ptr(), None,
                      stream(torch))
    got = host(pred)
    ref = OM.model_forward(SMALL, g, [], latents, O.timestep_embedding(np.array([0.3, 0.9], np.float32)), pe)
    assert max_abs_rel(got, ref) <= 1e-4
    mdl.free()


def _prefix_case(b, layers, seed):
    slots = [0] * 10 + [1] * 4 + [0] * 6      # text 16 + one 4x4 condition image
    shapes, target = [(4, 4)], (4, 8)
    ids, plen, tlen = O.joint_layout(len(slots), slots, shapes, target)
    pe = O.rope_table([(1, h, w) for h, w in shapes + [target]], [i >= 0 for i in ids])
    pieces = qimm.joint_layout_pieces(len(slots), slots, shapes)
    rng = np.random.default_rng(seed)
    txt = rng.standard_normal((b, len(slots), JD)).astype(np.float32)
    cond = rng.standard_normal((b, 16, CH)).astype(np.float32)
    key_valid = np.ones((b, plen), np.uint8)
    if b > 1:
        key_valid[1, 29:32] = 0                 # pad the last three text keys of row 1 (joint positions 29..31)
    return slots, ids[:plen], plen, pe[:plen], pieces, txt, cond, key_valid


def test_prefix_fill_matches_oracle(torch_cuda, qctx):
    torch = torch_cuda
    b, layers = 2, 2
    g, blocks = model_weights(31, layers)
    slots, ids, P, pe, pieces, txt, cond, key_valid = _prefix_case(b, layers, 6)
    assert P == 32 and all(i < 0 for i in ids[29:32]) and ids[10] == 0
    mdl = Built(qctx, g, blocks)
    kv = qctx.kv_create(layers, b, SMALL["heads"], P)
    txt_d, cond_d, pe_d = dev(torch, txt), dev(torch, cond), dev(torch, pe)
    ids_d, kv_d = dev(torch, np.array(ids, np.int32)), dev(torch, key_valid)
    mdl.model.prefix_fill(txt_d.data_ptr(), len(slots), cond_d.data_ptr(), 16, b, pieces, ids_d.data_ptr(),
                          kv_d.data_ptr(), pe_d.data_ptr(), kv, stream(torch))
    ref = OM.prefix_fill(SMALL, g, blocks, txt, cond, pieces, ids, key_valid, pe, mode=O.CANDLE)
    shape = (b, SMALL["heads"], P, 128)
    for i in range(layers):
        ko = torch.empty(shape, dtype=torch.int16, device="cuda")
        vo = torch.empty_like(ko)
        kv.load(i, ko.data_ptr(), vo.data_ptr(), stream(torch))
        k, v = O.bf16_to_f32(host(ko).view(np.uint16)), O.bf16_to_f32(host(vo).view(np.uint16))
        kr, vr = O.bf16_to_f32(ref[i][0]), O.bf16_to_f32(ref[i][1])
        assert cos_sim(k, kr) >= 0.9999 and max_abs_rel(k, kr) <= 2e-2, (i, cos_sim(k, kr), max_abs_rel(k, kr))
        assert cos_sim(v, vr) >= 0.9999 and max_abs_rel(v, vr) <= 2e-2, (i, cos_sim(v, vr), max_abs_rel(v, vr))
    kv.free()
    mdl.free()


def test_sampling_loop_with_cfg(torch_cuda, qctx):
    """Three steps of the T2I loop (src/pipeline.rs:168-193): prefix fill for the
    prompt and the negative prompt, then per step the cached forward twice, the
    CFG combine and the Euler update, all on the device."""
    torch = torch_cuda
    layers, T, sh, sw, steps, scale = 2, 12, 4, 8, 3, 4.0
    s = sh * sw
    g, blocks = model_weights(41, layers)
    rng = np.random.default_rng(9)
    txt = [rng.standard_normal((1, T, JD)).astype(np.float32) for _ in range(2)]
    latents = rng.standard_normal((1, s, CH)).astype(np.float32)
    ids, plen, _ = O.joint_layout(T, None, (), (sh, sw))
    pe_full = O.rope_table([(1, sh, sw)], [i >= 0 for i in ids])
    pieces = qimm.joint_layout_pieces(T)
    sig = qimm.flow_match_sigmas(steps, s)
    mdl = Built(qctx, g, blocks)
    caches = []
    keep = []
    for j in range(2):
        kv = qctx.kv_create(layers, 1, SMALL["heads"], plen)
        td, ped, idd = dev(torch, txt[j]), dev(torch, pe_full[:plen]), dev(torch, np.array(ids[:plen], np.int32))
        keep += [td, ped, idd]
        mdl.model.prefix_fill(td.data_ptr(), T, None, 0, 1, pieces, idd.data_ptr(), None, ped.data_ptr(), kv,
                              stream(torch))
        caches.append(kv)
    lat = dev(torch, latents)
    pe_t = dev(torch, pe_full[plen:])
    pc, pn = (torch.empty((1, s, CH), dtype=torch.float32, device="cuda") for _ in range(2))
    for i in range(steps):
        tsd = t_sin_dev(torch, qctx, [sig[i]])
        mdl.model.forward(lat.data_ptr(), 1, s, tsd.data_ptr(), pe_t.data_ptr(), caches[0], pc.data_ptr(), None,
                          stream(torch))
        mdl.model.forward(lat.data_ptr(), 1, s, tsd.data_ptr(), pe_t.data_ptr(), caches[1], pn.data_ptr(), None,
                          stream(torch))
        qctx.cfg_combine(pc.data_ptr(), pn.data_ptr(), s * CH, scale, pc.data_ptr(), stream(torch))
        qctx.euler_step(lat.data_ptr(), pc.data_ptr(), s * CH, OM.euler_dt(sig, i), stream(torch))
    got = host(lat)
    # the oracle loop
    ref_cache = [OM.prefix_fill(SMALL, g, blocks, txt[j], None, pieces, ids[:plen], None, pe_full[:plen])
                 for j in range(2)]
    x = latents.copy()
    for i in range(steps):
        ts = O.timestep_embedding(np.array([sig[i]], np.float32))
        preds = [OM.model_forward(SMALL, g, blocks, x, ts, pe_full[plen:], [k for k, _ in rc], [v for _, v in rc])
                 for rc in ref_cache]
        x = x + OM.cfg_combine(preds[0], preds[1], np.float32(scale)) * np.float32(OM.euler_dt(sig, i))
    assert cos_sim(got, x) >= 0.9999 and max_abs_rel(got, x) <= 2e-2, (cos_sim(got, x), max_abs_rel(got, x))
    upd, upd_r = got - latents, x - latents
    assert cos_sim(upd, upd_r) >= 0.999
    for kv in caches:
        kv.free()
    mdl.free()


def test_model_rejects_bad_calls(torch_cuda, qctx):
    g, blocks = model_weights(51, 1)
    keep = []
    blk = qctx.block_create(qimm.BlockConfig(SMALL["hidden"], SMALL["heads"], 128, SMALL["mlp"]),
                            block_tensors(blocks[0], keep))
    T = qimm.ModelTensors()
    t, data, rows, cols = g["img_in"]
    T.img_in = qimm.make_tensor(t, rows, cols, data.tobytes(), keep)  # the rest missing
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_ARG"):
        qctx.model_create(qimm.ModelConfig(CH, 0, SMALL["hidden"], 1), T, [blk])
    for name in ("t_linear_1", "t_linear_2", "modulation", "norm_out", "proj_out"):
        t, data, rows, cols = g[name]
        setattr(T, name, qimm.make_tensor(t, rows, cols, data.tobytes(), keep))
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):  # hidden differs from the block's
        qctx.model_create(qimm.ModelConfig(CH, 0, 2 * SMALL["hidden"], 1), T, [blk])
    m = qctx.model_create(qimm.ModelConfig(CH, 0, SMALL["hidden"], 1), T, [blk])
    kv = qctx.kv_create(1, 1, SMALL["heads"], 8)
    pe = torch_cuda.zeros((8, 128), dtype=torch_cuda.float32, device="cuda")
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):  # pieces do not cover the prefix
        m.prefix_fill(None, 0, None, 0, 1, [], None, None, pe.data_ptr(), kv)
    kv.free()
    m.free()
    blk.free()


def test_model_full_size_prefix_fill_and_forward(torch_cuda, qctx):
    """The step around the blocks at the reference's sizes (src/transformer.rs:63-79,
    src/quantized_transformer.rs:36-81,213-228,288-310,359-392,471-551): hidden 4096,
    32 heads, MLP 12288, joint dim 4096; the 256-token text prefix through txt_in
    (RMSNorm + 1, GELU-tanh) and two Q4_K_M blocks under the t = 0 modulation into
    the cache, then the cached forward of 4096 image tokens (img_in, the modulation
    GEMV [16384 x 4096], the blocks, norm_out, proj_out). Sampled rows of the
    prediction against oracle/model.py (blocks in candle mode, as the GPU blocks'
    default): cosine >= 0.9999, max|a-b|/max|b| <= 2e-2; the cache layers against the
    oracle's prefix pass."""
    torch = torch_cuda
    hid, heads, mlp, jd, ch, T, grid, layers = 4096, 32, 12288, 4096, 64, 256, 64, 2
    cfg = dict(hidden=hid, heads=heads, head_dim=128, mlp=mlp)
    s = grid * grid
    print("case: model forward hidden 4096, joint dim 4096, 2 blocks, 4096 tokens over a 256-token prefix",
          flush=True)
    rng = np.random.default_rng(77)
    g = {"img_in": synth.weight(rng, synth.F32, hid, ch, std=0.2),
         "t_linear_1": synth.weight(rng, synth.Q8_0, hid, 256, std=0.05),
         "t_linear_2": synth.weight(rng, synth.Q4_K, hid, hid, std=0.02),
         "modulation": synth.weight(rng, synth.Q4_K, 4 * hid, hid, std=0.02),
         "norm_out": synth.weight(rng, synth.BF16, hid, hid, std=0.02),
         "proj_out": synth.weight(rng, synth.Q6_K, ch, hid, std=0.02),
         "txt_norm": synth.weight(rng, synth.F32, 1, jd, std=0.1),
         "txt_in": synth.weight(rng, synth.Q8_0, hid, jd, std=0.02),
         "txt_out": synth.weight(rng, synth.Q8_0, hid, hid, std=0.02)}
    blocks = [synth.block_weights(780 + i, hid, heads, mlp, synth.Q4_K, synth.Q6_K) for i in range(layers)]
    keep = []
    blk = [qctx.block_create(qimm.BlockConfig(hid, heads, 128, mlp), block_tensors(w, keep)) for w in blocks]
    Tm = qimm.ModelTensors()
    for name, (t, data, rows, cols) in g.items():
        setattr(Tm, name, qimm.make_tensor(t, rows, cols, data.tobytes(), keep))
    model = qctx.model_create(qimm.ModelConfig(ch, jd, hid, layers), Tm, blk)
    txt = rng.standard_normal((1, T, jd)).astype(np.float32)
    latents = rng.standard_normal((1, s, ch)).astype(np.float32)
    ids, plen, _ = O.joint_layout(T, None, (), (grid, grid))
    pe_full = O.rope_table([(1, grid, grid)], [i >= 0 for i in ids])
    pieces = qimm.joint_layout_pieces(T)
    kv = qctx.kv_create(layers, 1, heads, plen)
    td, ped, idd = dev(torch, txt), dev(torch, pe_full[:plen]), dev(torch, np.array(ids[:plen], np.int32))
    model.prefix_fill(td.data_ptr(), T, None, 0, 1, pieces, idd.data_ptr(), None, ped.data_ptr(), kv, stream(torch))
    tsd = t_sin_dev(torch, qctx, [0.55])
    lat, pe_t = dev(torch, latents), dev(torch, pe_full[plen:])
    pred = torch.empty((1, s, ch), dtype=torch.float32, device="cuda")
    model.forward(lat.data_ptr(), 1, s, tsd.data_ptr(), pe_t.data_ptr(), kv, pred.data_ptr(), None, stream(torch))
    got = host(pred).reshape(s, ch)
    kg = torch.empty((1, heads, plen, 128), dtype=torch.bfloat16, device="cuda")
    vg = torch.empty_like(kg)
    cache = []
    for i in range(layers):
        kv.load(i, kg.data_ptr(), vg.data_ptr(), stream(torch))
        cache.append((host(kg.float()), host(vg.float())))
    kv.free()
    model.free()
    for b_ in blk:
        b_.free()
    assert np.isfinite(got).all()
    ref_cache = OM.prefix_fill(cfg, g, blocks, txt, None, pieces, ids[:plen], None, pe_full[:plen])
    for (k, v), (kr, vr) in zip(cache, ref_cache):
        for a, r in ((k, O.bf16_to_f32(kr)), (v, O.bf16_to_f32(vr))):
            assert cos_sim(a, r) >= 0.9999 and max_abs_rel(a, r) <= 2e-2, (cos_sim(a, r), max_abs_rel(a, r))
    rows = np.unique(np.concatenate([np.arange(4), np.random.default_rng(78).choice(s, 60, replace=False),
                                     np.arange(s - 4, s)]))
    ts = O.timestep_embedding(np.array([0.55], np.float32))
    ref = OM.model_forward_rows(cfg, g, blocks, latents, ts, pe_full[plen:], rows, [k for k, _ in ref_cache],
                                [v for _, v in ref_cache])
    c, m = cos_sim(got[rows], ref), max_abs_rel(got[rows], ref)
    print(f"prediction rows: cos {c:.7f} mar {m:.2e}", flush=True)
    assert c >= 0.9999 and m <= 2e-2
