"""The host side of the denoising step (N2) on the CPU: the sigma schedule
(FlowMatchEuler::new, src/scheduler.rs:24-37), the joint layout's prefix pieces
(JointLayout::new / assemble, src/joint_layout.rs:52-126), and the pinning of
the oracle's outer-model pieces (oracle/model.py)."""
import numpy as np
import pytest

import model as OM
import oracle as O
import qimm
import synth


# ---- sigmas: ports of src/scheduler.rs:148-185, plus independent checks ----

@pytest.mark.parametrize("seq", [64, 1024, 4096])
def test_schedule_endpoints_and_monotone(seq):
    for s in (qimm.flow_match_sigmas(20, seq), OM.flow_match_sigmas(20, seq)):
        s = list(s)
        assert len(s) == 20
        assert abs(s[0] - 1.0) < 1e-5
        assert abs(s[-1] - 0.02) < 1e-4
        assert all(a > b for a, b in zip(s, s[1:]))


def test_higher_resolution_shifts_more():
    assert qimm.flow_match_sigmas(20, 4096)[10] > qimm.flow_match_sigmas(20, 256)[10]
    assert OM.flow_match_sigmas(20, 4096)[10] > OM.flow_match_sigmas(20, 256)[10]


def test_single_step_schedule_is_nan_as_in_the_reference():
    # one step: the last sigma is 1, so stretch_shift_to_terminal's scale is 0 and
    # (1 - s) / scale is 0 / 0 (src/scheduler.rs:84-91)
    assert np.isnan(qimm.flow_match_sigmas(1, 256)[0]) and np.isnan(OM.flow_match_sigmas(1, 256)[0])


@pytest.mark.parametrize("steps,seq", [(2, 4096), (20, 256), (20, 4096), (50, 8192), (8, 100)])
def test_sigmas_library_oracle_closed_form(steps, seq):
    lib = np.array(qimm.flow_match_sigmas(steps, seq), np.float64)
    orc = OM.flow_match_sigmas(steps, seq).astype(np.float64)
    assert np.abs(lib - orc).max() <= 2e-7
    # the exponential shift written another way, in f64: t e^mu / (t e^mu + 1 - t),
    # mu linear in the token count through (256, 0.5) and (8192, 0.9)
    mu = 0.5 + (seq - 256) * (0.4 / (8192 - 256))
    t = np.linspace(1.0, 1.0 / steps, steps)
    sh = t * np.exp(mu) / (t * np.exp(mu) + 1.0 - t)
    sh = 1.0 - (1.0 - sh) * (1.0 - 0.02) / (1.0 - sh[-1])
    assert np.abs(lib - sh).max() <= 2e-6
    # the Euler steps telescope: sum(dt) = -sigma_0
    assert abs(sum(OM.euler_dt(lib, i) for i in range(steps)) + lib[0]) < 1e-6


# ---- prefix pieces: ports of src/joint_layout.rs:133-164 ----

def test_pieces_text_only():
    assert qimm.joint_layout_pieces(3) == [(0, 0, 3)]


def test_pieces_condition_slots_expand_in_place():
    # "a <pad><pad> b" with one 2x4-latent condition image (8 tokens = 2 slots)
    assert qimm.joint_layout_pieces(4, [0, 1, 1, 0], [(2, 4)]) == [(0, 0, 1), (1, 0, 8), (0, 3, 1)]


def test_pieces_adjacent_images_stay_separate():
    assert qimm.joint_layout_pieces(2, [1, 1], [(2, 2), (2, 2)]) == [(1, 0, 4), (1, 4, 4)]


@pytest.mark.parametrize("slots,shapes", [([0] * 5 + [1] * 6 + [0] * 9, [(4, 6)]),
                                          ([1] * 4 + [0] * 3 + [1] * 2 + [0], [(4, 4), (2, 4)]),
                                          ([0] * 7, [])])
def test_pieces_match_layout_ids(slots, shapes):
    pieces = qimm.joint_layout_pieces(len(slots), slots, shapes)
    ids, plen, _ = O.joint_layout(len(slots), slots, shapes, (2, 2))
    got, k = [], 0
    for kind, st, n in pieces:
        if kind == 0:
            got += [-1] * n
        else:
            got += [k] * n
            k += 1
    assert got == ids[:plen]
    # text pieces walk the non-slot prompt rows in order
    text_rows = [r for kind, st, n in pieces if kind == 0 for r in range(st, st + n)]
    assert text_rows == [i for i, s in enumerate(slots) if not s]


def test_pieces_reject_bad_layouts():
    with pytest.raises(qimm.QimmError):
        qimm.joint_layout_pieces(4, [0, 1, 1, 0], [])           # slots without an image
    with pytest.raises(qimm.QimmError):
        qimm.joint_layout_pieces(4, [0, 1, 0, 0], [(2, 4)])     # too few slots


# ---- oracle pinning ----

def test_activation_identities():
    x = np.linspace(-8, 8, 101)
    for f in (OM.silu, OM.gelu_tanh):
        assert np.allclose(f(x) - f(-x), x, atol=1e-12)
        assert f(np.array([0.0]))[0] == 0.0
    assert abs(OM.gelu_tanh(np.array([1.0]))[0] - 0.8411919906082768) < 1e-12  # tanh-form GELU(1)


def test_zero_timestep_embedding_constant():
    # zero_modulation feeds the constant [cos 0 ..., sin 0 ...] (src/quantized_transformer.rs:336-340)
    z = O.timestep_embedding(np.array([0.0], np.float32))
    assert np.array_equal(z, OM.zero_sinusoid(1))


# ---- timestep embedding: closed forms of src/scheduler.rs:101-126 ----

def _angles(t):
    return 1000.0 * np.float64(t) * 10000.0 ** (-np.arange(128) / 128.0)


@pytest.mark.parametrize("t", [0.001, 0.3, 0.97, 1.0])
def test_timestep_embedding_closed_form(t):
    """[cos(1000 t f_i) | sin(1000 t f_i)], f_i = 10000^(-i/128): cos first, the
    1000 time factor, exponent i/128 (not i/127). The tolerance covers the f32
    argument at t = 1 (angles up to 1000 rad, a few ulp each)."""
    got = O.timestep_embedding(np.array([t], np.float32))[0].astype(np.float64)
    a = _angles(np.float32(t))
    assert np.abs(got[:128] - np.cos(a)).max() <= 3e-4
    assert np.abs(got[128:] - np.sin(a)).max() <= 3e-4


def test_timestep_embedding_known_points():
    e = O.timestep_embedding(np.array([0.001, np.pi / 2000, 1e-6], np.float32)).astype(np.float64)
    # t = 0.001: the first angle is exactly 1 rad
    assert abs(e[0, 0] - np.cos(1.0)) < 1e-6 and abs(e[0, 128] - np.sin(1.0)) < 1e-6
    # t = pi/2000: the first angle is pi/2
    assert abs(e[1, 0]) < 1e-6 and abs(e[1, 128] - 1.0) < 1e-6
    # tiny t: cos half ~ 1, sin half ~ the angles themselves, which fall by 10000^(-1/128) per index
    assert np.all(np.abs(e[2, :128] - 1.0) < 1e-6)
    ratio = e[2, 129:256] / e[2, 128:255]
    assert np.allclose(ratio, 10000.0 ** (-1 / 128), rtol=1e-4)


def test_timestep_embedding_angles_recovered():
    # t = 0.003: every angle lies in (0, 3], so atan2 recovers it without wrapping
    e = O.timestep_embedding(np.array([0.003], np.float32))[0].astype(np.float64)
    ang = np.arctan2(e[128:], e[:128])
    assert np.allclose(ang, _angles(np.float32(0.003)), rtol=2e-6, atol=1e-7)


# ---- oracle/model.py compositions: special weights with closed-form outputs ----

def _f32w(mat):
    mat = np.ascontiguousarray(mat, dtype=np.float32)
    return (synth.F32, mat.view(np.uint8).ravel(), mat.shape[0], mat.shape[1])


def test_time_embed_identity_weights_is_silu():
    # linear_2(silu(linear_1(t))) with identity linears = silu(t) (src/quantized_transformer.rs:50-54)
    rng = np.random.default_rng(60)
    t = rng.standard_normal((3, 256)).astype(np.float32)
    g = {"t_linear_1": _f32w(np.eye(256)), "t_linear_2": _f32w(np.eye(256))}
    got = OM.time_embed(g, t)
    want = t.astype(np.float64) / (1.0 + np.exp(-t.astype(np.float64)))
    assert np.abs(got - want).max() < 1e-6


def test_modulation_chunks_and_silu():
    # Modulation::forward = silu(t_emb) . W^T (:226-228), [B, 1, 4h]; W rows [I; 2I; 0; -I]
    rng = np.random.default_rng(61)
    h = 64
    temb = rng.standard_normal((2, h)).astype(np.float32)
    eye = np.eye(h)
    g = {"modulation": _f32w(np.concatenate([eye, 2 * eye, 0 * eye, -eye]))}
    got = OM.modulation(g, temb)
    s = temb.astype(np.float64) / (1.0 + np.exp(-temb.astype(np.float64)))
    assert got.shape == (2, 1, 4 * h)
    want = np.concatenate([s, 2 * s, 0 * s, -s], axis=-1)[:, None, :]
    assert np.abs(got - want).max() < 1e-6


@pytest.mark.parametrize("stored", [0.0, 0.25])
def test_text_embedder_closed_form(stored):
    """QTextEmbedder (:76-81) with identity in/out layers: gelu_tanh(x / rms(x) * (1 + stored)),
    the stored norm weight being scale - 1 (ZeroCenterRMSNorm). An erf GELU or a missing
    +1 fails this."""
    rng = np.random.default_rng(62)
    d = 64
    x = (3.0 * rng.standard_normal((2, 5, d))).astype(np.float32)
    g = {"txt_norm": _f32w(np.full((1, d), stored)), "txt_in": _f32w(np.eye(d)), "txt_out": _f32w(np.eye(d))}
    got = OM.txt_in(g, x)
    xd = x.astype(np.float64)
    z = xd / np.sqrt((xd ** 2).mean(-1, keepdims=True) + 1e-6) * (1.0 + stored)
    want = 0.5 * z * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (z + 0.044715 * z ** 3)))
    assert np.abs(got - want).max() < 2e-6


@pytest.mark.parametrize("c", [0.0, 1.5, -0.5])
def test_final_layer_scale_after_layernorm(c):
    """FinalLayer (:300-309) + proj_out: LN(h) * (1 + linear(silu(t_emb))). With
    proj_out = I and a norm_out weight that maps silu(t_emb) to the constant c,
    every output row has mean 0 and standard deviation |1 + c|; scaling before the
    norm, or skipping the silu, gives another spread."""
    rng = np.random.default_rng(63)
    hid = 64
    h = (2.0 * rng.standard_normal((2, 7, hid)) + 0.5).astype(np.float32)
    t0 = 1.25
    temb = np.zeros((2, hid), np.float32)
    temb[:, 0] = t0
    w = np.zeros((hid, hid))
    w[:, 0] = c / (t0 / (1.0 + np.exp(-t0)))
    g = {"norm_out": _f32w(w), "proj_out": _f32w(np.eye(hid))}
    out = OM.final_layer(g, h, temb).astype(np.float64)
    assert np.abs(out.mean(-1)).max() < 1e-5
    assert np.abs(out.std(-1) - abs(1.0 + c)).max() < 1e-4


def test_model_forward_without_blocks():
    """With no blocks, identity img_in / proj_out and a zero norm_out the cached
    forward (:471-551) returns LayerNorm(latents); with proj_out zero it returns
    zero velocity."""
    rng = np.random.default_rng(64)
    ch, hid = 64, 64
    lat = rng.standard_normal((1, 9, ch)).astype(np.float32)
    t_sin = O.timestep_embedding(np.array([0.4], np.float32))
    g = {"img_in": _f32w(np.eye(hid)), "t_linear_1": _f32w(rng.standard_normal((hid, 256)) * 0.1),
         "t_linear_2": _f32w(np.eye(hid)), "modulation": _f32w(np.zeros((4 * hid, hid))),
         "norm_out": _f32w(np.zeros((hid, hid))), "proj_out": _f32w(np.eye(hid))}
    out = OM.model_forward(dict(hidden=hid), g, [], lat, t_sin, None).astype(np.float64)
    ld = lat.astype(np.float64)
    want = (ld - ld.mean(-1, keepdims=True)) / np.sqrt(ld.var(-1, keepdims=True) + 1e-6)
    assert np.abs(out - want).max() < 1e-5
    g["proj_out"] = _f32w(np.zeros((ch, hid)))
    assert not OM.model_forward(dict(hidden=hid), g, [], lat, t_sin, None).any()


def test_model_forward_rows_equal_full_forward():
    """The rows variant (every block but the last in full, the last through
    block_forward_rows, the final layer per row) gives the listed rows of the
    full forward bit for bit: two blocks, batch 2, a prefix cache, rows across
    the batch boundary and unsorted."""
    cfg = dict(hidden=256, heads=2, head_dim=128, mlp=512)
    rng = np.random.default_rng(5)
    h, ch, b, s, p = 256, 16, 2, 12, 8
    g = {"img_in": synth.weight(rng, synth.F32, h, ch, std=0.2),
         "t_linear_1": synth.weight(rng, synth.Q8_0, h, 256, std=0.05),
         "t_linear_2": synth.weight(rng, synth.Q8_0, h, h, std=0.05),
         "modulation": synth.weight(rng, synth.Q8_0, 4 * h, h, std=0.05),
         "norm_out": synth.weight(rng, synth.F32, h, h, std=0.05),
         "proj_out": synth.weight(rng, synth.F32, ch, h, std=0.05)}
    blocks = [synth.block_weights(70 + i, h, 2, 512, synth.Q4_K, synth.Q6_K) for i in range(2)]
    lat = rng.standard_normal((b, s, ch)).astype(np.float32)
    ts = O.timestep_embedding(np.array([0.3, 0.8], np.float32))
    pe = O.rope_table([(1, 3, 4)], [1] * s)
    kc = [O.f32_to_bf16(rng.standard_normal((b, 2, p, 128))) for _ in range(2)]
    vc = [O.f32_to_bf16(rng.standard_normal((b, 2, p, 128))) for _ in range(2)]
    full = OM.model_forward(cfg, g, blocks, lat, ts, pe, kc, vc).reshape(b * s, ch)
    rows = np.array([17, 0, 11, 12, 5, 23])
    part = OM.model_forward_rows(cfg, g, blocks, lat, ts, pe, rows, kc, vc)
    assert np.array_equal(part.view(np.uint32), full[rows].view(np.uint32))
