"""GPU parity of the prefix fill and the masked attention it runs on.

The prefix pass (QwenImageTransformer::prefix_kv, src/quantized_transformer.rs:359-392)
runs every block over the text + condition tokens with the block-causal mask
(build_block_causal_mask, src/attention_mask.rs:18-66) and the text key
validity (key_valid, :349-356); the uncached full sequence (:508-543) runs the
same mask with per-token modulation rows; the cached step passes only
key_valid. Through qimm_attention_masked and qimm_block_forward_masked, against
the oracle on identical seeded inputs, with the bars of the other GPU tests:
cosine >= 0.9999 and max|a-b|/max|b| <= 2e-2. The cache invariant of
src/bin/kv_cache_probe.rs (cached step == the target rows of the uncached
sequence) is checked GPU against GPU with the same bars.
"""
import numpy as np
import pytest

import oracle as O
import synth
from gpu_util import bf16_dev, cos_sim, dev, host, max_abs_rel, stream
from test_gpu_block import SMALL, block_tensors

import qimm

pytestmark = pytest.mark.gpu


def _layout(text_slots, cond_shapes, target):
    """image ids of a joint sequence, its prefix length and the RoPE table over it."""
    ids, plen, tlen = O.joint_layout(len(text_slots), text_slots, cond_shapes, target)
    pe = O.rope_table([(1, h, w) for h, w in list(cond_shapes) + [target]], [i >= 0 for i in ids])
    return np.array(ids, dtype=np.int64), plen, tlen, pe


# text 5, condition image 4x6 (6 slots), text 9 | target 4x8: prefix 38, total 70
LAYOUT_SMALL = ([0] * 5 + [1] * 6 + [0] * 9, [(4, 6)], (4, 8))
# text 10, condition image 8x8 (16 slots), text 30 | target 12x16: prefix 104, total 296
LAYOUT_MID = ([0] * 10 + [1] * 16 + [0] * 30, [(8, 8)], (12, 16))


def _key_valid(b, ids, pad_last_text):
    """batch row i pads the last pad_last_text[i] text keys of the prefix."""
    kv = np.ones((b, ids.size), dtype=np.uint8)
    text = np.nonzero(ids < 0)[0]
    for i, n in enumerate(pad_last_text):
        if n:
            kv[i, text[-n:]] = 0
    return kv


def _dense_mask(ids, kvalid):
    return O.block_causal_mask(ids)[None] * kvalid[:, None, :]


def _bhsd(torch, rng, b, h, s, mul=1.0):
    return bf16_dev(torch, (mul * rng.standard_normal((b, h, s, 128))).astype(np.float32))


def _vt(torch, v):
    d, _ = bf16_dev(torch, np.ascontiguousarray(v.transpose(0, 1, 3, 2)))
    return d


@pytest.mark.parametrize("layout,b,h,pads", [(LAYOUT_SMALL, 2, 2, (0, 3)), (LAYOUT_MID, 2, 3, (7, 0)),
                                             (LAYOUT_MID, 1, 2, (0,))])
def test_attention_block_causal_matches_oracle(torch_cuda, qctx, layout, b, h, pads):
    """Uncached full sequence: block-causal mask over [prefix ; target] plus key validity."""
    torch = torch_cuda
    ids, _, _, _ = _layout(*layout)
    s = ids.size
    rng = np.random.default_rng(s + b + h)
    q_dev, q = _bhsd(torch, rng, b, h, s)
    k_dev, k = _bhsd(torch, rng, b, h, s)
    _, v = _bhsd(torch, rng, b, h, s)
    kvalid = _key_valid(b, ids, pads)
    ids_dev = dev(torch, ids.astype(np.int32))
    kv_dev = dev(torch, kvalid)
    vt_dev = _vt(torch, v)
    out = torch.empty((b, s, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention_masked(q_dev.data_ptr(), b, h, s, None, 0, k_dev.data_ptr(), vt_dev.data_ptr(), s,
                          128 ** -0.5, out.data_ptr(), ids_dev.data_ptr(), kv_dev.data_ptr(), stream(torch))
    got = host(out.float()).reshape(b, s, h, 128).transpose(0, 2, 1, 3)
    want = O.attention(q, k, v, scale=128 ** -0.5, mask=_dense_mask(ids, kvalid), mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2, (cos_sim(got, want),
                                                                             max_abs_rel(got, want))


def test_attention_block_causal_without_key_valid(torch_cuda, qctx):
    torch = torch_cuda
    ids, _, _, _ = _layout(*LAYOUT_MID)
    s, b, h = ids.size, 1, 2
    rng = np.random.default_rng(5)
    q_dev, q = _bhsd(torch, rng, b, h, s, 3.0)
    k_dev, k = _bhsd(torch, rng, b, h, s)
    _, v = _bhsd(torch, rng, b, h, s)
    ids_dev = dev(torch, ids.astype(np.int32))
    vt_dev = _vt(torch, v)
    out = torch.empty((b, s, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention_masked(q_dev.data_ptr(), b, h, s, None, 0, k_dev.data_ptr(), vt_dev.data_ptr(), s,
                          128 ** -0.5, out.data_ptr(), ids_dev.data_ptr(), None, stream(torch))
    got = host(out.float()).reshape(b, s, h, 128).transpose(0, 2, 1, 3)
    want = O.attention(q, k, v, mask=O.block_causal_mask(ids)[None], mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2


@pytest.mark.parametrize("b,h,p,so,pads", [(2, 2, 38, 32, (0, 3)), (2, 2, 104, 192, (5, 1)), (1, 1, 70, 8, (9,))])
def test_attention_cached_step_key_valid(torch_cuda, qctx, b, h, p, so, pads):
    """Cached step: target queries see every valid prefix key and every own key."""
    torch = torch_cuda
    rng = np.random.default_rng(p + so)
    ids = np.array([-1] * p + [0] * so, dtype=np.int64)
    kvalid = _key_valid(b, ids, pads)
    q_dev, q = _bhsd(torch, rng, b, h, so)
    ko_dev, ko = _bhsd(torch, rng, b, h, so)
    _, vo = _bhsd(torch, rng, b, h, so)
    kp_dev, kp = _bhsd(torch, rng, b, h, p)
    vp_dev, vp = _bhsd(torch, rng, b, h, p)
    kv = qctx.kv_create(1, b, h, p)
    kv.store(0, kp_dev.data_ptr(), vp_dev.data_ptr(), stream(torch))
    kv_dev = dev(torch, kvalid)
    vt_dev = _vt(torch, vo)
    out = torch.empty((b, so, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention_masked(q_dev.data_ptr(), b, h, so, kv, 0, ko_dev.data_ptr(), vt_dev.data_ptr(), so,
                          128 ** -0.5, out.data_ptr(), None, kv_dev.data_ptr(), stream(torch))
    got = host(out.float()).reshape(b, so, h, 128).transpose(0, 2, 1, 3)
    kv.free()
    mask = np.broadcast_to(kvalid[:, None, :], (b, so, p + so))
    want = O.attention(q, ko, vo, kp, vp, mask=mask, mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2


def _masked_case(torch, qctx, ids, kvalid, h, rows=None, seed=0, qmul=1.0):
    """Prefix-less masked attention of ids.size tokens on the GPU and in the oracle (exact mode),
    on all rows or on the listed query rows."""
    b, s = kvalid.shape[0] if kvalid is not None else 1, ids.size
    rng = np.random.default_rng(seed)
    q_dev, q = _bhsd(torch, rng, b, h, s, qmul)
    k_dev, k = _bhsd(torch, rng, b, h, s)
    _, v = _bhsd(torch, rng, b, h, s)
    ids_dev = dev(torch, ids.astype(np.int32))
    kv_dev = dev(torch, kvalid) if kvalid is not None else None
    vt_dev = _vt(torch, v)
    out = torch.empty((b, s, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention_masked(q_dev.data_ptr(), b, h, s, None, 0, k_dev.data_ptr(), vt_dev.data_ptr(), s,
                          128 ** -0.5, out.data_ptr(), ids_dev.data_ptr(),
                          kv_dev.data_ptr() if kv_dev is not None else None, stream(torch))
    got = host(out.float()).reshape(b, s, h, 128).transpose(0, 2, 1, 3)
    rows = np.arange(s) if rows is None else np.asarray(rows)
    mask = O.block_causal_mask(ids)[rows][None]
    if kvalid is not None:
        mask = mask * kvalid[:, None, :]
    want = O.attention(np.ascontiguousarray(q[:, :, rows]), k, v, scale=128 ** -0.5, mask=mask, mode=O.EXACT)
    return got[:, :, rows], want


def _ids(*runs):
    """image ids from (id, count) runs; -1 = text."""
    return np.concatenate([np.full(n, i, dtype=np.int64) for i, n in runs])


@pytest.mark.parametrize("runs,b,pad", [
    (((-1, 40), (0, 256), (1, 256), (-1, 24), (2, 128)), 2, "last"),   # block edges off the 64-key grid
    (((-1, 16), (0, 64), (-1, 24), (1, 128)), 2, "first"),               # padding on the first keys
    (((-1, 24), (0, 40), (-1, 16), (0, 24), (1, 32)), 1, None),          # one id in two runs
    (((0, 96), (1, 96), (2, 64)), 1, None),                              # no text
    (((-1, 200),), 2, "first"),                                          # text only: causal
])
def test_attention_block_causal_fast_path(torch_cuda, qctx, runs, b, pad):
    """Every length a multiple of 8: the masked form of the fast kernel, with windows
    that run unmasked, skipped windows and windows tested score by score; rows whose
    first keys are padding start their softmax later."""
    ids = _ids(*runs)
    kvalid = None
    if pad:
        kvalid = np.ones((b, ids.size), dtype=np.uint8)
        text = np.nonzero(ids < 0)[0]
        if pad == "last":
            kvalid[-1, text[-9:]] = 0
        else:
            kvalid[-1, text[:5]] = 0
    got, want = _masked_case(torch_cuda, qctx, ids, kvalid, h=2, seed=ids.size + b)
    if pad == "first":
        # queries that see only padded keys have an all -inf row: NaN, as the
        # reference's softmax gives
        bad = np.isnan(want)
        assert np.array_equal(np.isnan(got), bad)
        got, want = np.where(bad, 0, got), np.where(bad, 0, want)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2, (cos_sim(got, want),
                                                                             max_abs_rel(got, want))


def test_attention_block_causal_prefix_8448(torch_cuda, qctx):
    """The multi-reference prefix: 256 text tokens and two 64 x 64 condition images
    (8448 tokens), sampled query rows around every block edge."""
    ids = _ids((-1, 256), (0, 4096), (1, 4096))
    rows = [0, 1, 63, 64, 200, 255, 256, 257, 1000, 4351, 4352, 4353, 6000, 8446, 8447]
    got, want = _masked_case(torch_cuda, qctx, ids, None, h=4, rows=rows, seed=8448)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2, (cos_sim(got, want),
                                                                             max_abs_rel(got, want))


@pytest.mark.parametrize("b,h,p,so", [(2, 2, 64, 64), (1, 3, 136, 256)])
def test_attention_cached_step_key_valid_fast_path(torch_cuda, qctx, b, h, p, so):
    """Cached step with key validity, both segments multiples of 8 (the fast kernel's
    masked form): padding at the start of the prefix and inside it."""
    torch = torch_cuda
    rng = np.random.default_rng(p + so + 1)
    kvalid = np.ones((b, p + so), dtype=np.uint8)
    kvalid[0, :70] = 0           # whole first window and part of the second
    kvalid[-1, 3:11] = 0
    q_dev, q = _bhsd(torch, rng, b, h, so)
    ko_dev, ko = _bhsd(torch, rng, b, h, so)
    _, vo = _bhsd(torch, rng, b, h, so)
    kp_dev, kp = _bhsd(torch, rng, b, h, p)
    vp_dev, vp = _bhsd(torch, rng, b, h, p)
    kv = qctx.kv_create(1, b, h, p)
    kv.store(0, kp_dev.data_ptr(), vp_dev.data_ptr(), stream(torch))
    kv_dev = dev(torch, kvalid)
    vt_dev = _vt(torch, vo)
    out = torch.empty((b, so, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention_masked(q_dev.data_ptr(), b, h, so, kv, 0, ko_dev.data_ptr(), vt_dev.data_ptr(), so,
                          128 ** -0.5, out.data_ptr(), None, kv_dev.data_ptr(), stream(torch))
    got = host(out.float()).reshape(b, so, h, 128).transpose(0, 2, 1, 3)
    kv.free()
    mask = np.broadcast_to(kvalid[:, None, :], (b, so, p + so))
    want = O.attention(q, ko, vo, kp, vp, mask=mask, mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2


def test_attention_masked_rejects_bad_calls(torch_cuda, qctx):
    torch = torch_cuda
    b, h, s = 1, 1, 16
    q = torch.zeros((b, h, s, 128), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((b, s, h * 128), dtype=torch.bfloat16, device="cuda")
    ids = dev(torch, np.zeros(s, dtype=np.int32))
    kv = qctx.kv_create(1, b, h, 8)
    with pytest.raises(qimm.QimmError, match="SHAPE"):  # image ids with a cached prefix
        qctx.attention_masked(q.data_ptr(), b, h, s, kv, 0, q.data_ptr(), q.data_ptr(), s, 0.1, out.data_ptr(),
                              ids.data_ptr(), None, stream(torch))
    with pytest.raises(qimm.QimmError, match="SHAPE"):  # image ids with so != sq
        qctx.attention_masked(q.data_ptr(), b, h, s, None, 0, q.data_ptr(), q.data_ptr(), s - 1, 0.1,
                              out.data_ptr(), ids.data_ptr(), None, stream(torch))
    kv.free()


# ---------------------------------------------------------------- block

def _block(torch, qctx, w):
    keep = []
    c = qimm.BlockConfig(SMALL["hidden"], SMALL["heads"], SMALL["head_dim"], SMALL["mlp"])
    return qctx.block_create(c, block_tensors(w, keep))


def _forward_masked(torch, qctx, blk, x, mod, pe, ids=None, kvalid=None, kv=None, want_kv=False):
    b, s, _ = x.shape
    H = SMALL["heads"]
    x_d, mod_d, pe_d = dev(torch, x), dev(torch, mod), dev(torch, pe)
    ids_d = dev(torch, ids.astype(np.int32)) if ids is not None else None
    kv_d = dev(torch, kvalid) if kvalid is not None else None
    out = torch.empty_like(x_d)
    k_out = torch.empty((b, H, s, 128), dtype=torch.bfloat16, device="cuda") if want_kv else None
    v_out = torch.empty_like(k_out) if want_kv else None
    blk.forward_masked(x_d.data_ptr(), out.data_ptr(), b, s, mod_d.data_ptr(), mod.shape[1], pe_d.data_ptr(),
                       ids_d.data_ptr() if ids_d is not None else None,
                       kv_d.data_ptr() if kv_d is not None else None, kv, 0,
                       k_out.data_ptr() if want_kv else None, v_out.data_ptr() if want_kv else None, stream(torch))
    return host(out), k_out, v_out


def _case(seed, b, layout, attn_type=synth.Q4_K, down_type=synth.Q6_K):
    rng = np.random.default_rng(seed)
    w = synth.block_weights(seed, SMALL["hidden"], SMALL["heads"], SMALL["mlp"], attn_type, down_type, True)
    ids, plen, tlen, pe = _layout(*layout)
    x = rng.standard_normal((b, ids.size, SMALL["hidden"])).astype(np.float32)
    mod0 = (rng.standard_normal((b, 1, 4 * SMALL["hidden"])) * 0.5).astype(np.float32)   # t = 0 rows
    mod1 = (rng.standard_normal((b, 1, 4 * SMALL["hidden"])) * 0.5).astype(np.float32)   # the step's rows
    return w, ids, plen, tlen, pe, x, mod0, mod1


def _check(got, ref):
    cs, mr = cos_sim(got, ref), max_abs_rel(got, ref)
    assert cs >= 0.9999 and mr <= 2e-2, (cs, mr)


@pytest.mark.parametrize("layout,b,pads,types", [(LAYOUT_SMALL, 2, (0, 3), (synth.Q4_K, synth.Q6_K)),
                                                 (LAYOUT_MID, 2, (4, 0), (synth.Q8_0, synth.Q8_0)),
                                                 (LAYOUT_MID, 1, (0,), (synth.Q6_K, synth.Q4_K))])
def test_block_prefix_pass_matches_oracle(torch_cuda, qctx, layout, b, pads, types):
    """prefix_kv: one block over the prefix rows, one modulation row, block-causal mask."""
    torch = torch_cuda
    w, ids, plen, _, pe, x, mod0, _ = _case(11 + b + len(layout[0]), b, layout, *types)
    xp, idp, pep = np.ascontiguousarray(x[:, :plen]), ids[:plen], pe[:plen]
    kvalid = _key_valid(b, idp, pads)
    blk = _block(torch, qctx, w)
    got, k, v = _forward_masked(torch, qctx, blk, xp, mod0, pep, idp, kvalid, want_kv=True)
    blk.free()
    ref, kr, vr = O.block_forward(SMALL, w, xp, mod0, pep, mask=_dense_mask(idp, kvalid), mode=O.CANDLE)
    _check(got, ref)
    _check(host(k.float()), kr)
    _check(host(v.float()), vr)


@pytest.mark.parametrize("layout,b,pads", [(LAYOUT_SMALL, 2, (0, 2)), (LAYOUT_MID, 1, (3,))])
def test_block_uncached_full_sequence_matches_oracle(torch_cuda, qctx, layout, b, pads):
    """Uncached step: per-token modulation rows (t = 0 rows for the prefix) and the full mask."""
    torch = torch_cuda
    w, ids, plen, tlen, pe, x, mod0, mod1 = _case(23 + b, b, layout)
    mod = np.concatenate([np.repeat(mod0, plen, 1), np.repeat(mod1, tlen, 1)], 1)
    kvalid = _key_valid(b, ids, pads)
    blk = _block(torch, qctx, w)
    got, _, _ = _forward_masked(torch, qctx, blk, x, mod, pe, ids, kvalid)
    blk.free()
    ref, _, _ = O.block_forward(SMALL, w, x, mod, pe, mask=_dense_mask(ids, kvalid), mode=O.CANDLE)
    _check(got, ref)


@pytest.mark.parametrize("layout,b,pads", [(LAYOUT_SMALL, 2, (0, 3)), (LAYOUT_MID, 1, (5,))])
def test_cached_step_equals_uncached_target_rows(torch_cuda, qctx, layout, b, pads):
    """kv_cache_probe invariant for one block: fill the cache with the prefix pass,
    then the cached step over the target rows matches those rows of the uncached
    full sequence."""
    torch = torch_cuda
    w, ids, plen, tlen, pe, x, mod0, mod1 = _case(31 + b, b, layout)
    kvalid = _key_valid(b, ids, pads)
    blk = _block(torch, qctx, w)
    _, k, v = _forward_masked(torch, qctx, blk, np.ascontiguousarray(x[:, :plen]), mod0, pe[:plen], ids[:plen],
                              np.ascontiguousarray(kvalid[:, :plen]), want_kv=True)
    kv = qctx.kv_create(1, b, SMALL["heads"], plen)
    kv.store(0, k.data_ptr(), v.data_ptr(), stream(torch))
    cached, _, _ = _forward_masked(torch, qctx, blk, np.ascontiguousarray(x[:, plen:]), mod1,
                                   np.ascontiguousarray(pe[plen:]), None, kvalid, kv=kv)
    mod = np.concatenate([np.repeat(mod0, plen, 1), np.repeat(mod1, tlen, 1)], 1)
    full, _, _ = _forward_masked(torch, qctx, blk, x, mod, pe, ids, kvalid)
    kv.free()
    blk.free()
    _check(cached, full[:, plen:])
    # and both against the oracle's cached step on the GPU's own prefix K/V
    kq = O.f32_to_bf16(host(k.float()))
    vq = O.f32_to_bf16(host(v.float()))
    ref, _, _ = O.block_forward(SMALL, w, np.ascontiguousarray(x[:, plen:]), mod1, np.ascontiguousarray(pe[plen:]),
                                kq, vq, mask=np.broadcast_to(kvalid[:, None, :], (b, tlen, plen + tlen)),
                                mode=O.CANDLE)
    _check(cached, ref)


@pytest.mark.parametrize("layout,b,pads", [(LAYOUT_SMALL, 2, (0, 3)), (LAYOUT_MID, 1, (0,))])
def test_attention_q8_0_rounding_in_epilogue_bit_identical(torch_cuda, qctx, monkeypatch, layout, b, pads):
    """The masked prefix pass with Q8_0 weights: the attention output's Q8_0
    rounding (to_out's input) done by the masked attention kernels' epilogue
    against the same rounding as the rows-quantizer pass
    (QIMM_SEPARATE_ROUNDING=1): bit-identical block outputs and k / v."""
    torch = torch_cuda
    w, ids, plen, _, pe, x, mod0, _ = _case(31 + b, b, layout, synth.Q8_0, synth.Q8_0)
    xp, idp, pep = np.ascontiguousarray(x[:, :plen]), ids[:plen], pe[:plen]
    kvalid = _key_valid(b, idp, pads)
    blk = _block(torch, qctx, w)
    got, k, v = _forward_masked(torch, qctx, blk, xp, mod0, pep, idp, kvalid, want_kv=True)
    monkeypatch.setenv("QIMM_SEPARATE_ROUNDING", "1")
    ref, kr, vr = _forward_masked(torch, qctx, blk, xp, mod0, pep, idp, kvalid, want_kv=True)
    blk.free()
    assert np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert torch.equal(k, kr) and torch.equal(v, vr)
