"""RoPE tables, rope_i and the joint layout: the reference's own unit tests
(src/rope.rs:278-316 and 351-361, src/joint_layout.rs:133-164) restated on
the oracle, and the product library's host-side restatements (qimm_rope_table,
qimm_joint_layout; CPU-only code) checked against the oracle bit for bit."""
import numpy as np
import pytest

import oracle as O

AXES = (16, 56, 56)


def closed_form(coord, axes=AXES, theta=10000.0):
    """coordinate * theta^(-2i/dim) per axis (src/rope.rs:256-268)."""
    cos, sin = [], []
    for a, dim in enumerate(axes):
        for i in range(dim // 2):
            ang = coord[a] * theta ** (-2.0 * i / dim)
            cos.append(np.cos(ang))
            sin.append(np.sin(ang))
    return np.array(cos), np.array(sin)


def test_embed_nd_matches_reference_formula():
    # src/rope.rs:278-316: text_len 2 + one (1, 2, 2) image block
    pe = O.rope_table([(1, 2, 2)], [0, 0, 1, 1, 1, 1])
    assert pe.shape == (6, 128)
    assert np.all((np.abs(np.abs(pe[0]) - 1) < 1e-4) | (np.abs(pe[0]) < 1e-4))
    for k, (h, w) in enumerate([(-1, -1), (-1, 0), (0, -1), (0, 0)]):
        c, s = closed_form((2, h, w))
        want = np.stack([c, s], axis=1).reshape(-1)
        assert np.max(np.abs(pe[2 + k] - want)) < 1e-3, (k, h, w)


def test_rope_positions_text_image_text():
    # text advances all axes; image freezes frame at the running position and
    # moves it by max(h, w); trailing text continues from there (src/rope.rs:125-172)
    mask = [0, 0, 0] + [1] * 12 + [0, 0]
    pe = O.rope_table([(1, 3, 4)], mask)
    c, s = closed_form((3, -2, -2))          # first image token: h0 = -(3-1) = -2, w0 = -(4-2) = -2
    assert np.max(np.abs(pe[3, 0::2] - c)) < 1e-3
    c, s = closed_form((3, 0, 1))            # last image token: h = 0, w = 1
    assert np.max(np.abs(pe[14, 1::2] - s)) < 1e-3
    c, s = closed_form((3 + 4, 7, 7))        # trailing text: p = 3 + max(3, 4)
    assert np.max(np.abs(pe[15, 0::2] - c)) < 1e-3


def test_apply_rope_matches_complex_multiply():
    # src/rope.rs:351-361: rope_i against the unfused complex product, tol 1e-5
    rng = np.random.default_rng(20)
    x = rng.standard_normal((1, 3, 5, 16)).astype(np.float32)
    ang = (rng.standard_normal((5, 8)) * 3).astype(np.float32)
    freqs = np.stack([np.cos(ang), np.sin(ang)], axis=2).reshape(5, 16).astype(np.float32)
    got = O.apply_rope(x, freqs)
    z = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * ang.astype(np.float64))
    want = np.stack([z.real, z.imag], axis=-1).reshape(x.shape)
    assert np.max(np.abs(got - want)) < 1e-5


def test_layout_text_only_is_text_then_target():
    ids, pl, tl = O.joint_layout(3, None, [], (2, 2))
    assert ids == [-1, -1, -1, 0, 0, 0, 0] and (pl, tl) == (3, 4)


def test_layout_condition_slots_expand_in_place():
    ids, pl, tl = O.joint_layout(4, [0, 1, 1, 0], [(2, 4)], (2, 2))
    assert ids == [-1] + [0] * 8 + [-1] + [1] * 4 and (pl, tl) == (10, 4)


def test_layout_adjacent_condition_images_stay_separate_blocks():
    ids, _, _ = O.joint_layout(2, [1, 1], [(2, 2), (2, 2)], (2, 2))
    assert ids[:8] == [0, 0, 0, 0, 1, 1, 1, 1]


@pytest.mark.parametrize("args", [
    (2, [1, 1], [], (2, 2)),              # more image slots than condition images
    (2, [0, 0], [(2, 2)], (2, 2)),        # condition image without slots
    (2, [1, 1], [(3, 3)], (2, 2)),        # h*w not a multiple of 4
    (3, [1, 0, 1], [(2, 4)], (2, 2)),     # slots not consecutive
])
def test_layout_errors(args):
    with pytest.raises(ValueError):
        O.joint_layout(*args)


def test_block_causal_mask_predicate():
    ids = [-1, -1, 0, 0, 0, -1, 1, 1]
    m = O.block_causal_mask(ids)
    for q in range(8):
        for k in range(8):
            want = q >= k or (ids[q] == ids[k] and ids[q] >= 0)
            assert bool(m[q, k]) == want


# ---- the product's host-side restatements (run on the CPU) ----

def _qimm():
    import qimm
    try:
        qimm.load()
    except (OSError, qimm.QimmError) as e:
        pytest.skip(f"libqimm.so not loadable here: {e}")
    return qimm


def test_product_rope_table_equals_oracle_bitwise():
    qimm = _qimm()
    mask = [0] * 7 + [1] * 48 + [0] * 3 + [1] * 16
    shapes = [(1, 6, 8), (1, 4, 4)]
    a = qimm.rope_table(shapes, mask)
    b = O.rope_table(shapes, mask)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_product_rope_table_t2i_1024():
    qimm = _qimm()
    mask = [0] * 256 + [1] * 4096
    a = qimm.rope_table([(1, 64, 64)], mask)
    b = O.rope_table([(1, 64, 64)], mask)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("args", [
    (3, None, [], (2, 2)),
    (4, [0, 1, 1, 0], [(2, 4)], (2, 2)),
    (2, [1, 1], [(2, 2), (2, 2)], (2, 2)),
    (300, [0] * 10 + [1] * 256 + [0] * 34, [(32, 32)], (64, 64)),
])
def test_product_joint_layout_equals_oracle(args):
    qimm = _qimm()
    assert qimm.joint_layout(*args) == O.joint_layout(*args)


def test_product_joint_layout_errors():
    qimm = _qimm()
    with pytest.raises(qimm.QimmError):
        qimm.joint_layout(2, [1, 1], [], (2, 2))
