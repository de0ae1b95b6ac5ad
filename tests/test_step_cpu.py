"""The host side of the denoising step (N2) on the CPU: the sigma schedule
(FlowMatchEuler::new, src/scheduler.rs:24-37), the joint layout's prefix pieces
(JointLayout::new / assemble, src/joint_layout.rs:52-126), and the pinning of
the oracle's outer-model pieces (oracle/model.py)."""
import numpy as np
import pytest

import model as OM
import oracle as O
import qimm


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
