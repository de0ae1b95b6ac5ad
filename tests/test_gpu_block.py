"""GPU parity of the whole block step (TransformerBlock::forward on the cached
step, src/quantized_transformer.rs:258-285) through qimm_block_create /
qimm_block_forward, against the oracle on identical seeded inputs, in both
activation modes of the block (gpu_util.check_block):
- QIMM_ACT_CANDLE (the default: the reference CPU path's int8 rounding of every
  quantized-matmul input) against the oracle's candle mode: the output reaches
  cosine >= 0.9999 and max|a-b|/max|b| <= 2e-2, and its update x_out - x lies
  at least as close to candle's as the bf16 mode's does;
- QIMM_ACT_BF16 against the oracle's exact mode (f32 activations, f64
  accumulation): cosine >= 0.9999 on the output and on the stricter update,
  max|a-b|/max|b| <= 2e-2.
The own k / v the block returns are checked against the matching oracle mode.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
import qimm
import synth
from gpu_util import check_block, cos_sim, dev, host, kv_close, max_abs_rel, stream

pytestmark = pytest.mark.gpu


def block_tensors(w, keep):
    T = qimm.BlockTensors()
    for name, field in (("to_q", "to_q"), ("to_k", "to_k"), ("to_v", "to_v"), ("to_out", "to_out"),
                        ("gate_up", "gate_up"), ("proj", "proj"), ("gate_layer", "gate_layer"),
                        ("down", "mlp_out")):
        if name in w:
            t, data, rows, cols = w[name]
            setattr(T, field, qimm.make_tensor(t, rows, cols, data.tobytes(), keep))
    for name in ("norm_q", "norm_k"):
        arr = np.ascontiguousarray(w[name], dtype=np.float32)
        setattr(T, name, qimm.make_tensor(synth.F32, arr.size, 1, arr.tobytes(), keep))
    return T


def run_block(torch, qctx, cfg, w, x, mod, pe, kpre=None, vpre=None, alias=False, want_kv=False,
              act=qimm.ACT_CANDLE):
    keep = []
    c = qimm.BlockConfig(cfg["hidden"], cfg["heads"], cfg["head_dim"], cfg["mlp"])
    blk = qctx.block_create(c, block_tensors(w, keep))
    assert blk.act_mode == qimm.ACT_CANDLE  # the default
    blk.set_act_mode(act)
    b, s, hid = x.shape
    x_dev = dev(torch, x)
    x_out = x_dev if alias else torch.empty_like(x_dev)
    kv = None
    mod_d, pe_d = dev(torch, mod), dev(torch, pe)  # device buffers stay referenced until the step ran
    if kpre is not None:
        kv = qctx.kv_create(3, b, cfg["heads"], kpre.shape[2])
        k_d, v_d = dev(torch, kpre.view(np.int16)), dev(torch, vpre.view(np.int16))
        kv.store(2, k_d.data_ptr(), v_d.data_ptr(), stream(torch))
    k_out = v_out = None
    if want_kv:
        k_out = torch.empty((b, cfg["heads"], s, 128), dtype=torch.bfloat16, device="cuda")
        v_out = torch.empty_like(k_out)
    blk.forward(x_dev.data_ptr(), x_out.data_ptr(), b, s, mod_d.data_ptr(), pe_d.data_ptr(),
                kv, 2, k_out.data_ptr() if want_kv else None, v_out.data_ptr() if want_kv else None, stream(torch))
    out = host(x_out)
    kvs = (host(k_out.float()), host(v_out.float())) if want_kv else (None, None)
    blk.free()
    if kv is not None:
        kv.free()
    return out, kvs


def run_modes(torch, qctx, cfg, w, x, mod, pe, kpre=None, vpre=None, alias=False, want_kv=False):
    """The block in the candle and the bf16 activation mode: ((out, kv), (out, kv))."""
    return tuple(run_block(torch, qctx, cfg, w, x, mod, pe, kpre, vpre, alias, want_kv, act)
                 for act in (qimm.ACT_CANDLE, qimm.ACT_BF16))


def check_modes(cfg, w, x, mod, pe, kpre, vpre, runs, want_kv=False):
    """Both modes' outputs (and own k / v) against the oracle's matching modes."""
    (got_c, kv_c), (got_b, kv_b) = runs
    ref, kr, vr = O.block_forward(cfg, w, x, mod, pe, kpre, vpre, mode=O.CANDLE)
    ref_e, kre, vre = O.block_forward(cfg, w, x, mod, pe, kpre, vpre, mode=O.EXACT)
    hid = cfg["hidden"]
    check_block(*(a.reshape(-1, hid) for a in (got_c, got_b, ref, ref_e, x)))
    if want_kv:
        for (k, v), (kk, vv) in ((kv_c, (kr, vr)), (kv_b, (kre, vre))):
            kv_close(k, kk)
            kv_close(v, vv)


def make_case(seed, cfg, b, s, p, attn_type, down_type, fused=True):
    rng = np.random.default_rng(seed)
    w = synth.block_weights(seed, cfg["hidden"], cfg["heads"], cfg["mlp"], attn_type, down_type, fused)
    x = rng.standard_normal((b, s, cfg["hidden"])).astype(np.float32)
    mod = (rng.standard_normal((b, 1, 4 * cfg["hidden"])) * 0.5).astype(np.float32)
    gh = int(np.sqrt(s))
    while s % gh:
        gh -= 1
    pe = O.rope_table([(1, gh, s // gh)], [0] * p + [1] * s)[p:]
    kpre = vpre = None
    if p:
        kpre = O.f32_to_bf16(rng.standard_normal((b, cfg["heads"], p, 128)))
        vpre = O.f32_to_bf16(rng.standard_normal((b, cfg["heads"], p, 128)))
    return w, x, mod, pe, kpre, vpre


SMALL = dict(hidden=256, heads=2, head_dim=128, mlp=768)


def check(got, ref, x, exact=False):
    """exact=False: cosine on the output; exact=True: cosine on the update."""
    cs = cos_sim(got - x, ref - x) if exact else cos_sim(got, ref)
    mr = max_abs_rel(got, ref)
    assert cs >= 0.9999 and mr <= 2e-2, (cs, mr)


@pytest.mark.parametrize("attn_type,down_type", [(synth.Q8_0, synth.Q8_0), (synth.Q4_K, synth.Q6_K),
                                                 (synth.Q6_K, synth.Q4_K)])
@pytest.mark.parametrize("b,s,p", [(1, 16, 8), (2, 24, 16),  # M <= 64: split-K weight-streaming GEMM
                                   (1, 96, 40), (2, 64, 64), (1, 130, 0),
                                   # M >= 512 takes the 256x256 GEMM: partial tiles, a batch
                                   # boundary inside a tile, S % 4 != 0, and sequences shorter
                                   # than a tile (three in one tile)
                                   (1, 520, 24), (2, 300, 16), (1, 514, 0), (3, 200, 8)])
def test_block_matches_oracle(torch_cuda, qctx, attn_type, down_type, b, s, p):
    w, x, mod, pe, kpre, vpre = make_case(b * 1000 + s + p, SMALL, b, s, p, attn_type, down_type)
    runs = run_modes(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre, want_kv=True)
    check_modes(SMALL, w, x, mod, pe, kpre, vpre, runs, want_kv=True)


def test_block_in_place_and_separate_mlp_inputs(torch_cuda, qctx):
    w, x, mod, pe, kpre, vpre = make_case(7, SMALL, 1, 64, 16, synth.Q8_0, synth.Q8_0, fused=False)
    runs = run_modes(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre, alias=True)
    check_modes(SMALL, w, x, mod, pe, kpre, vpre, runs)


def test_block_mixed_qkv_types_unfused_path(torch_cuda, qctx):
    """to_v in Q8_0 beside Q4_K to_q / to_k: unfused q/k/v GEMMs, and in candle
    mode the norm1 output rounded per 256 values for q and k, per 32 for v."""
    w, x, mod, pe, kpre, vpre = make_case(8, SMALL, 1, 64, 32, synth.Q4_K, synth.Q6_K)
    rng = np.random.default_rng(80)
    w["to_v"] = synth.weight(rng, synth.Q8_0, SMALL["hidden"], SMALL["hidden"])
    runs = run_modes(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre, want_kv=True)
    check_modes(SMALL, w, x, mod, pe, kpre, vpre, runs, want_kv=True)


def test_block_large_norm_weights_running_max_path(torch_cuda, qctx):
    """q/k RmsNorm weights of magnitude ~3 (a score bound of ~150 in log2 units,
    above the attention's fixed-reference limit of 64): the attention keeps the
    running maximum; the small-weight cases elsewhere take the fixed reference.
    Both modes against the oracle, with a prefix cache and without."""
    for p in (32, 0):
        w, x, mod, pe, kpre, vpre = make_case(13 + p, SMALL, 1, 96, p, synth.Q4_K, synth.Q6_K)
        rng = np.random.default_rng(131 + p)
        w["norm_q"] = (3.0 + 0.3 * rng.standard_normal(128)).astype(np.float32)
        w["norm_k"] = (3.0 + 0.3 * rng.standard_normal(128)).astype(np.float32)
        runs = run_modes(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre, want_kv=True)
        check_modes(SMALL, w, x, mod, pe, kpre, vpre, runs, want_kv=True)


def test_block_deterministic(torch_cuda, qctx):
    w, x, mod, pe, kpre, vpre = make_case(9, SMALL, 1, 96, 32, synth.Q4_K, synth.Q6_K)
    a, _ = run_block(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre)
    b, _ = run_block(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre)
    assert np.array_equal(a, b)


def test_block_config1_shape(torch_cuda, qctx):
    """Hidden 3072, 24 heads x 128, MLP 9216, 256 image tokens over a 64-token
    prefix, Q8_0 weights: the reference CPU-path configuration."""
    cfg = dict(hidden=3072, heads=24, head_dim=128, mlp=9216)
    w, x, mod, pe, kpre, vpre = make_case(11, cfg, 1, 256, 64, synth.Q8_0, synth.Q8_0)
    runs = run_modes(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    check_modes(cfg, w, x, mod, pe, kpre, vpre, runs)


@pytest.mark.parametrize("b,s,p,mlp", [(1, 8, 16, 512), (2, 6, 0, 1024), (2, 8, 8, 1024), (1, 16, 0, 2048),
                                       (2, 20, 8, 1024), (1, 64, 16, 1024),
                                       # MLP 12288: gate_up (24576 x 4096) keeps six groups per CU over the
                                       # whole K (SwiGLU epilogue at 40 and at 2 x 12 tokens)
                                       (1, 40, 16, 12288), (2, 12, 8, 12288)])
def test_block_hidden4096_short_m(torch_cuda, qctx, b, s, p, mlp):
    """Hidden 4096 (32 heads) at M <= 64 tokens: the fused QKV (12288 x 4096),
    output (4096 x 4096) and gate_up (2 mlp x 4096) projections and, for
    mlp % 1024 == 0, the Q6_K down projection take the one-launch kernel with
    its q/k/v (RmsNorm + RoPE + layouts, batch boundaries inside the token
    tile), residual and SwiGLU epilogues; mlp 512 sends the down projection to
    the split-K dequantizing kernel. Short MLPs keep the oracle quick; the
    model's MLP 12288 runs at 40 and 24 tokens."""
    cfg = dict(hidden=4096, heads=32, head_dim=128, mlp=mlp)
    w, x, mod, pe, kpre, vpre = make_case(21 + b + s, cfg, b, s, p, synth.Q4_K, synth.Q6_K)
    runs = run_modes(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre, want_kv=True)
    check_modes(cfg, w, x, mod, pe, kpre, vpre, runs, want_kv=True)


@pytest.mark.parametrize("b,s,p,mlp,attn_type,down_type", [
    (1, 1028, 16, 1024, synth.Q4_K, synth.Q6_K),  # a 4-row last tile row
    (2, 520, 8, 1024, synth.Q4_K, synth.Q6_K),    # batch boundary inside the third 256-row tile
    (1, 1024, 0, 2048, synth.Q8_0, synth.Q8_0),   # four full tile rows, no prefix
    (1, 2820, 0, 4096, synth.Q4_K, synth.Q6_K)])  # out, gate_up and down on 256 x 256 tiles too
def test_block_hidden4096_large_m(torch_cuda, qctx, b, s, p, mlp, attn_type, down_type):
    """Hidden 4096 (32 heads) at M >= 1024 tokens, where the q/k/v projection
    has enough 256 x 256 tiles for the large-M GEMM: its fused q/k/v epilogue
    over 32 heads (head = column / 128 across 48 column tiles, V written
    transposed) and the XCD-aware tile order, with partial tiles and a batch
    boundary inside a tile; at 2820 tokens (12 tile rows) also its residual
    (out, Q6_K down) and SwiGLU epilogues, on a 4-row last tile row. The
    products with fewer tiles take the 128 x 128 kernel. Output, k and v against
    both oracle modes. Short MLPs keep the oracle quick."""
    cfg = dict(hidden=4096, heads=32, head_dim=128, mlp=mlp)
    w, x, mod, pe, kpre, vpre = make_case(61 + b + s, cfg, b, s, p, attn_type, down_type)
    runs = run_modes(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre, want_kv=True)
    check_modes(cfg, w, x, mod, pe, kpre, vpre, runs, want_kv=True)


def test_block_hidden4096_large_m_bf16_weights(torch_cuda, qctx):
    """Float-stored (bf16) weights at 2820 tokens, hidden 4096, MLP 4096: the
    large-M GEMM's bf16 form, whose weight tile goes global -> LDS by direct
    loads like the activations, under its fused q/k/v, residual and SwiGLU
    epilogues (12 tile rows, a 4-row last one). Candle multiplies float-stored
    weights in plain f32 (no int8 activations), so exact mode alone is the
    reference here."""
    cfg = dict(hidden=4096, heads=32, head_dim=128, mlp=4096)
    b, s, p = 1, 2820, 0
    w, x, mod, pe, kpre, vpre = make_case(67, cfg, b, s, p, synth.BF16, synth.BF16)
    got, (k, v) = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre, want_kv=True)
    ref_e, kre, vre = O.block_forward(cfg, w, x, mod, pe, kpre, vpre, mode=O.EXACT)
    check(got, ref_e, x)
    check(got, ref_e, x, exact=True)
    assert cos_sim(k, kre) >= 0.9999 and max_abs_rel(k, kre) <= 2e-2
    assert cos_sim(v, vre) >= 0.9999 and max_abs_rel(v, vre) <= 2e-2


@pytest.mark.parametrize("attn_type,down_type", [(synth.Q8_0, synth.Q8_0), (synth.Q4_K, synth.Q6_K)])
def test_block_mid_m_split_k(torch_cuda, qctx, attn_type, down_type):
    """Hidden 1024 (8 heads), MLP 2048, 128 tokens over a 16-token prefix: every
    projection's 128x128 tiles leave CUs idle, so each runs split over K (2
    shares of whole 512-value groups) with its partial sums added by the q/k/v,
    SwiGLU and residual epilogues of the reduction kernel."""
    cfg = dict(hidden=1024, heads=8, head_dim=128, mlp=2048)
    w, x, mod, pe, kpre, vpre = make_case(31, cfg, 1, 128, 16, attn_type, down_type)
    runs = run_modes(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre, want_kv=True)
    check_modes(cfg, w, x, mod, pe, kpre, vpre, runs, want_kv=True)
    again, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    assert np.array_equal(runs[0][0], again)


def test_block_rejects_bad_config(torch_cuda, qctx):
    keep = []
    w = synth.block_weights(1, 256, 2, 768, synth.Q8_0)
    bad = qimm.BlockConfig(256, 4, 64, 768)   # head_dim 64 unsupported
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        qctx.block_create(bad, block_tensors(w, keep))
    c = qimm.BlockConfig(256, 2, 128, 768)
    T = block_tensors(w, keep)
    T.to_q = qimm.make_tensor(synth.Q8_0, 256, 256, b"\0" * 100, keep)   # wrong byte count
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        qctx.block_create(c, T)


def test_block_reserve_then_forward(torch_cuda, qctx):
    """qimm_block_reserve pre-sizes the context scratch: forwards at the reserved
    size and below give the same bits as forwards that grow the scratch themselves,
    and bad sizes are rejected."""
    w, x, mod, pe, kpre, vpre = make_case(12, SMALL, 1, 96, 16, synth.Q4_K, synth.Q6_K)
    a, _ = run_block(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre)
    keep = []
    blk = qctx.block_create(qimm.BlockConfig(256, 2, 128, 768), block_tensors(w, keep))
    blk.reserve(2, 600)
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        blk.reserve(1, 64, 3)
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_ARG"):
        blk.set_act_mode(2)
    blk.free()
    b, _ = run_block(torch_cuda, qctx, SMALL, w, x, mod, pe, kpre, vpre)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("case", ["config1_128x128", "wide_ragged", "two_k_shares"])
def test_hidden_q8_0_rounding_in_gate_up_epilogue_bit_identical(torch_cuda, qctx, monkeypatch, case):
    """Q8_0 down weights in candle mode: the Q8_0 rounding of the SwiGLU hidden
    state (the down projection's input, one scale per 32 columns of a token row)
    done by the gate_up kernel's epilogue against the same rounding as the
    rows-quantizer pass (QIMM_SEPARATE_ROUNDING=1): bit-identical block outputs.
    Cases: config 1 (MLP 9216 at 256 tokens over 64: the undivided 128x128
    kernel, four lanes per block), hidden 1024 / MLP 4096 at 1100 tokens (the
    256x256 kernel, two waves per block, a last token tile of 76 rows), and the
    same block at 256 tokens (two K shares: the f32 state and the rows quantizer
    on both sides)."""
    if case == "config1_128x128":
        cfg, b, s, p = dict(hidden=3072, heads=24, head_dim=128, mlp=9216), 1, 256, 64
    else:
        cfg, b, s, p = dict(hidden=1024, heads=8, head_dim=128, mlp=4096), 1, 1100 if case == "wide_ragged" else 256, 64
    print(f"case: {case}, hidden {cfg['hidden']}, MLP {cfg['mlp']}, {s} tokens", flush=True)
    w, x, mod, pe, kpre, vpre = make_case(43, cfg, b, s, p, synth.Q8_0, synth.Q8_0)
    fused, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    monkeypatch.setenv("QIMM_SEPARATE_ROUNDING", "1")
    separate, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    assert np.isfinite(fused).all()
    diff = np.count_nonzero(fused.view(np.uint32) != separate.view(np.uint32))
    print(f"{case}: outputs differing in any bit: {diff} of {fused.size}", flush=True)
    assert diff == 0


@pytest.mark.parametrize("case", ["config1_fast_4wave", "ragged_any_length"])
def test_attention_q8_0_rounding_in_epilogue_bit_identical(torch_cuda, qctx, monkeypatch, case):
    """Q8_0 weights in candle mode: the attention output's Q8_0 rounding (to_out's
    input, 32 values of one head per block) done by the attention kernel's
    epilogue against the same rounding as the rows-quantizer pass
    (QIMM_SEPARATE_ROUNDING=1): bit-identical block outputs. Cases: config 1
    (hidden 3072, 24 heads, MLP 9216, 256 tokens over 64: the 4-wave fast
    kernel) and a prefix and token count that are not multiples of 8 (the
    any-length kernel)."""
    if case == "config1_fast_4wave":
        cfg, b, s, p = dict(hidden=3072, heads=24, head_dim=128, mlp=9216), 1, 256, 64
    else:
        cfg, b, s, p = SMALL, 2, 100, 61
    w, x, mod, pe, kpre, vpre = make_case(41, cfg, b, s, p, synth.Q8_0, synth.Q8_0)
    fused, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    monkeypatch.setenv("QIMM_SEPARATE_ROUNDING", "1")
    separate, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    assert np.isfinite(fused).all()
    diff = np.count_nonzero(fused.view(np.uint32) != separate.view(np.uint32))
    print(f"{case}: outputs differing in any bit: {diff} of {fused.size}", flush=True)
    assert diff == 0
