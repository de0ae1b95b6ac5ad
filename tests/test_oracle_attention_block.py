"""Pins the oracle's attention and block.

Attention: numpy float64 softmax attention (library matmul and exp) on random
inputs; special cases (a single key returns its value, identical keys return
the mean of V); prefix-split invariance; masking.
Block: the reference's KV-cache invariant (src/bin/kv_cache_probe.rs:53-70):
the uncached full-sequence pass with the block-causal mask and t=0 prefix rows
gives the same target rows as the cached target-only pass over the bf16 prefix
cache; and an independent numpy float64 composition of the block on a tiny
config, written from src/quantized_transformer.rs:124-285 in array form.
"""
import numpy as np
import pytest

import oracle as O
import synth


def np_attention(q, k, v, scale, mask=None):
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), k.astype(np.float64)) * scale
    if mask is not None:
        s = np.where(mask[:, None, :, :] != 0, s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("bhij,bhjd->bhid", p, v.astype(np.float64))


@pytest.mark.parametrize("mode,tol", [(O.EXACT, 1e-6), (O.CANDLE, 2e-5)])
def test_attention_matches_numpy(mode, tol):
    rng = np.random.default_rng(30)
    b, h, sq, p, so, d = 2, 3, 17, 11, 17, 32
    q = rng.standard_normal((b, h, sq, d)).astype(np.float32)
    kp, vp = rng.standard_normal((2, b, h, p, d)).astype(np.float32)
    ko, vo = rng.standard_normal((2, b, h, so, d)).astype(np.float32)
    got = O.attention(q, ko, vo, kp, vp, mode=mode)
    want = np_attention(q, np.concatenate([kp, ko], 2), np.concatenate([vp, vo], 2), d ** -0.5)
    assert np.max(np.abs(got - want)) < tol


def test_attention_single_key_returns_value():
    rng = np.random.default_rng(31)
    q = rng.standard_normal((1, 2, 5, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 1, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 1, 16)).astype(np.float32)
    out = O.attention(q, k, v, mode=O.CANDLE)
    assert np.array_equal(out, np.broadcast_to(v, out.shape))


def test_attention_identical_keys_give_mean_of_values():
    rng = np.random.default_rng(32)
    q = rng.standard_normal((1, 1, 4, 16)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 1, 16)).astype(np.float32), 9, axis=2)
    v = rng.standard_normal((1, 1, 9, 16)).astype(np.float32)
    out = O.attention(q, k, v, mode=O.EXACT)
    assert np.allclose(out, np.broadcast_to(v.mean(axis=2, keepdims=True), out.shape), atol=1e-6)


def test_attention_prefix_split_invariance():
    rng = np.random.default_rng(33)
    q = rng.standard_normal((1, 2, 8, 16)).astype(np.float32)
    k = rng.standard_normal((1, 2, 20, 16)).astype(np.float32)
    v = rng.standard_normal((1, 2, 20, 16)).astype(np.float32)
    whole = O.attention(q, k, v, mode=O.EXACT)
    split = O.attention(q, k[:, :, 7:], v[:, :, 7:], k[:, :, :7], v[:, :, :7], mode=O.EXACT)
    assert np.allclose(whole, split, atol=1e-7)


def test_attention_mask_matches_numpy():
    rng = np.random.default_rng(34)
    ids = [-1] * 5 + [0] * 6 + [1] * 4
    s = len(ids)
    mask = O.block_causal_mask(ids)[None]
    q, k, v = rng.standard_normal((3, 1, 2, s, 8)).astype(np.float32)
    got = O.attention(q, k, v, mask=mask, mode=O.EXACT)
    want = np_attention(q, k, v, 8 ** -0.5, mask)
    assert np.max(np.abs(got - want)) < 1e-6


# ---------------------------------------------------------------- block

CFG = dict(hidden=256, heads=2, head_dim=128, mlp=768)


def tiny_inputs(seed, s, t_prefix=0, wtype=O.Q8_0, down=None, fused=True):
    rng = np.random.default_rng(seed)
    w = synth.block_weights(seed, CFG["hidden"], CFG["heads"], CFG["mlp"], wtype, down, fused)
    x = rng.standard_normal((1, s, CFG["hidden"])).astype(np.float32)
    mod = (rng.standard_normal((1, 1, 4 * CFG["hidden"])) * 0.5).astype(np.float32)
    return w, x, mod, rng


def np_block(w, x, mod, pe, kpre=None, vpre=None):
    """float64 array-form restatement of TransformerBlock::forward with exact weights."""
    hid, H, D, F = CFG["hidden"], CFG["heads"], CFG["head_dim"], CFG["mlp"]
    W = {n: O.dequantize(t, data, r * c).reshape(r, c).astype(np.float64)
         for n, (t, data, r, c) in ((k, v) for k, v in w.items() if isinstance(v, tuple))}
    x = x.astype(np.float64)
    s1, g1, s2, g2 = np.split(mod.astype(np.float64), 4, axis=-1)

    def ln(t):
        mu = t.mean(-1, keepdims=True)
        return (t - mu) / np.sqrt(((t - mu) ** 2).mean(-1, keepdims=True) + 1e-6)

    def rms(t, g):
        return t / np.sqrt((t ** 2).mean(-1, keepdims=True) + 1e-6) * g

    def rope(t):
        c, sn = pe[:, 0::2].astype(np.float64), pe[:, 1::2].astype(np.float64)
        a, b = t[..., 0::2], t[..., 1::2]
        return np.stack([a * c - b * sn, a * sn + b * c], -1).reshape(t.shape)

    b_, s = x.shape[:2]
    n1 = ln(x) * (1 + s1)
    q = (n1 @ W["to_q"].T).reshape(b_, s, H, D)
    k = (n1 @ W["to_k"].T).reshape(b_, s, H, D)
    v = (n1 @ W["to_v"].T).reshape(b_, s, H, D).transpose(0, 2, 1, 3)
    q = rope(rms(q, w["norm_q"]).transpose(0, 2, 1, 3))
    k = rope(rms(k, w["norm_k"]).transpose(0, 2, 1, 3))
    ka, va = k, v
    if kpre is not None:
        ka = np.concatenate([O.bf16_to_f32(kpre).astype(np.float64), k], 2)
        va = np.concatenate([O.bf16_to_f32(vpre).astype(np.float64), v], 2)
    att = np_attention(q, ka, va, D ** -0.5).transpose(0, 2, 1, 3).reshape(b_, s, hid)
    x1 = x + np.tanh(g1) * (att @ W["to_out"].T)
    n2 = ln(x1) * (1 + s2)
    gu = n2 @ W["gate_up"].T
    gate, up = gu[..., :F], gu[..., F:]
    hm = gate / (1 + np.exp(-gate)) * up
    return x1 + np.tanh(g2) * (hm @ W["down"].T)


def cos_sim(a, b):
    a, b = a.astype(np.float64).ravel(), b.astype(np.float64).ravel()
    return a @ b / np.sqrt((a @ a) * (b @ b))


@pytest.mark.parametrize("wtype,down", [(O.Q8_0, None), (O.Q4_K, O.Q6_K)])
def test_block_exact_mode_matches_numpy_composition(wtype, down):
    s, p = 24, 8
    w, x, mod, rng = tiny_inputs(40, s, wtype=wtype, down=down)
    pe = O.rope_table([(1, 4, 6)], [0] * p + [1] * s)[p:]
    kpre = O.f32_to_bf16(rng.standard_normal((1, 2, p, 128)))
    vpre = O.f32_to_bf16(rng.standard_normal((1, 2, p, 128)))
    got, _, _ = O.block_forward(CFG, w, x, mod, pe, kpre, vpre, mode=O.EXACT)
    want = np_block(w, x, mod, pe, kpre, vpre)
    assert np.max(np.abs(got - want)) < 1e-4 * np.abs(want).max()


def test_block_candle_mode_close_to_exact():
    s = 32
    w, x, mod, _ = tiny_inputs(41, s)
    pe = O.rope_table([(1, 4, 8)], [1] * s)
    a, _, _ = O.block_forward(CFG, w, x, mod, pe, mode=O.CANDLE)
    b, _, _ = O.block_forward(CFG, w, x, mod, pe, mode=O.EXACT)
    assert cos_sim(a - x, b - x) > 0.999


def test_block_separate_proj_gate_equals_fused():
    s = 16
    w, x, mod, _ = tiny_inputs(42, s)
    F = CFG["mlp"]
    t, data, rows, cols = w["gate_up"]
    rb = O.row_bytes(t, cols)
    ws = {k: v for k, v in w.items() if k != "gate_up"}
    ws["gate_layer"] = (t, data[: F * rb], F, cols)
    ws["proj"] = (t, data[F * rb:], F, cols)
    pe = O.rope_table([(1, 4, 4)], [1] * s)
    a, _, _ = O.block_forward(CFG, w, x, mod, pe)
    b, _, _ = O.block_forward(CFG, ws, x, mod, pe)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("mode", [O.CANDLE, O.EXACT])
def test_block_cached_equals_uncached(mode):
    """kv_cache_probe's invariant on one block."""
    p, gh, gw = 12, 4, 5
    s = gh * gw
    w, x_img, mod_img, rng = tiny_inputs(43, s)
    x_txt = rng.standard_normal((1, p, CFG["hidden"])).astype(np.float32)
    mod_zero = (rng.standard_normal((1, 1, 4 * CFG["hidden"])) * 0.5).astype(np.float32)
    ids, pl, tl = O.joint_layout(p, None, [], (gh, gw))
    pe_full = O.rope_table([(1, gh, gw)], [0] * p + [1] * s)
    mask = O.block_causal_mask(ids)[None]
    x_full = np.concatenate([x_txt, x_img], 1)
    mod_full = np.concatenate([np.repeat(mod_zero, p, 1), np.repeat(mod_img, s, 1)], 1)
    out_full, k_full, v_full = O.block_forward(CFG, w, x_full, mod_full, pe_full, mask=mask, mode=mode)
    # the prefix pass alone (prefix rows, t=0 row, causal mask) gives the cache
    out_pre, k_pre, v_pre = O.block_forward(CFG, w, x_txt, mod_zero, pe_full[:p],
                                            mask=O.block_causal_mask(ids[:p])[None], mode=mode)
    assert np.allclose(k_pre, k_full[:, :, :p], atol=1e-5)
    kc, vc = O.f32_to_bf16(k_pre), O.f32_to_bf16(v_pre)
    out_cached, _, _ = O.block_forward(CFG, w, x_img, mod_img, pe_full[p:], kc, vc, mode=mode)
    ref = out_full[:, p:]
    assert cos_sim(out_cached - x_img, ref - x_img) > 0.99999
    assert np.max(np.abs(out_cached - ref)) / np.max(np.abs(ref)) < 1e-3


@pytest.mark.parametrize("mode", [O.CANDLE, O.EXACT])
@pytest.mark.parametrize("per_token_mod,masked,fused", [(False, False, True), (True, True, False),
                                                        (False, True, True)])
def test_block_rows_equal_full_block_rows(mode, per_token_mod, masked, fused):
    """oq_block_forward_rows (query side for a subset of token rows) against the
    full forward: bit-identical rows and K/V, over two batch entries, a prefix,
    per-token modulation rows, a block-causal mask and the separate proj/gate
    MLP; the rows come unsorted and straddle the batch boundary."""
    b, s, p = 2, 20, 6
    w, _, _, rng = tiny_inputs(44, s, fused=fused)
    x = rng.standard_normal((b, s, CFG["hidden"])).astype(np.float32)
    mod = (rng.standard_normal((b, s if per_token_mod else 1, 4 * CFG["hidden"])) * 0.5).astype(np.float32)
    pe = O.rope_table([(1, 4, 5)], [0] * p + [1] * s)[p:]
    kpre = O.f32_to_bf16(rng.standard_normal((b, 2, p, 128)))
    vpre = O.f32_to_bf16(rng.standard_normal((b, 2, p, 128)))
    mask = None
    if masked:
        mask = (rng.random((b, s, p + s)) < 0.7).astype(np.uint8)
        mask[:, :, p] = 1   # every query keeps at least one key
    full, kf, vf = O.block_forward(CFG, w, x, mod, pe, kpre, vpre, mask=mask, mode=mode)
    rows = np.array([27, 3, 0, 19, 20, 39, 11])
    got, kr, vr = O.block_forward_rows(CFG, w, x, mod, pe, rows, kpre, vpre, mask=mask, mode=mode)
    assert np.array_equal(got, full.reshape(b * s, -1)[rows])
    assert np.array_equal(kr, kf) and np.array_equal(vr, vf)


def test_exact_gemm_is_row_and_tile_independent():
    """Exact mode's f64 sums depend on the output's own row and column only:
    any row subset, odd M and N and a K that is not a multiple of 4 (f32
    weights) give bit-identical outputs, equal to numpy's f64 product up to the
    final rounding to f32."""
    rng = np.random.default_rng(45)
    for t, n, k in ((O.F32, 37, 75), (O.Q8_0, 70, 96), (O.Q4_K, 33 * 4, 512)):
        m = 67
        x = rng.standard_normal((m, k)).astype(np.float32)
        if t == O.F32:
            w = rng.standard_normal((n, k)).astype(np.float32).view(np.uint8).ravel()
        else:
            _, w, _, _ = synth.weight(rng, t, n, k)
        y = O.qmatmul(t, w, n, k, x, O.EXACT)
        rows = np.array([66, 0, 33, 5])
        assert np.array_equal(O.qmatmul(t, w, n, k, x[rows], O.EXACT), y[rows])
        want = x.astype(np.float64) @ O.dequantize(t, w, n * k).reshape(n, k).astype(np.float64).T
        assert np.max(np.abs(y - want)) <= 1e-6 * np.abs(want).max()
