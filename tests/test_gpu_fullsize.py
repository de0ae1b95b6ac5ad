"""GPU parity at the reference's full shapes, through the C ABI.

- The 1024x1024 block step with Q4_K_M weights: hidden 4096, 32 heads x 128,
  MLP 12288, 4096 image tokens (64 x 64 latent grid) over a cached 256-token
  bf16 text prefix; q/k/v/out/gate_up in Q4_K, the down projection in Q6_K
  (TransformerBlock::forward, src/quantized_transformer.rs:258-285, at the
  sizes of src/transformer.rs:63-88). This runs the 256 x 256 GEMM with its
  fused q/k/v (32 heads), SwiGLU (N = 24576) and residual (Q6_K, K = 12288)
  epilogues and its XCD-aware tile order, on 16 x 16..96 tiles.
- The image-conditioned multi-reference step with true CFG: batch 2 (the two
  prompts), 4096 target tokens over an 8448-token cached prefix each (256 text
  + 2 condition images of 64 x 64 latents), 12544 keys; Q8_0 weights
  (src/quantized_transformer.rs:143-148, src/pipeline.rs:154-155,178-186).
- The Q8_0 dequant-GEMM sets at 4352 and 256 tokens: fused QKV 12288 x 4096,
  out 4096 x 4096, MLP up 16384 x 4096 and down 4096 x 16384
  (src/quantized_transformer.rs:19-33).

Bars (gpu_util.check_block). The block in its default QIMM_ACT_CANDLE mode
(every quantized-matmul input rounded to int8 as the reference CPU path does:
Q8_K per 256 values for K-quant weights, Q8_0 per 32 for Q8_0) against the
oracle's candle mode: cosine >= 0.9999 and max|a-b|/max|b| <= 2e-2 on the
output (at 1024^2 over all rows, and on each row by itself), its update x_out - x closer to
candle's than the bf16 mode's update. The block in QIMM_ACT_BF16 mode against
the oracle's exact mode (f32 activations, f64 sums of the exact weights):
cosine >= 0.9999 on the output and on the update, max|a-b|/max|b| <= 2e-2, and
closer to exact arithmetic than the candle path. (At hidden 4096 with MLP
12288 the candle path itself is only at cosine ~0.99988 from exact
arithmetic: its int8 rounding of the SwiGLU hidden state alone accounts for
most of that, so each mode is held to the reference whose rounding it follows.)
Where the oracle would take minutes, the query side runs for sampled token rows
only (oracle.block_forward_rows: every row's K and V, bit-identical rows).
"""
import numpy as np
import pytest

import oracle as O
import qimm
import synth
from gpu_util import bf16_dev, check_block, cos_sim, kv_close, max_abs_rel, host, stream
from test_gpu_block import make_case, run_block, run_modes
from test_gpu_kernels import _attention_case

pytestmark = pytest.mark.gpu

CFG4 = dict(hidden=4096, heads=32, head_dim=128, mlp=12288)


def sampled_rows(rng, m, tile=256, extra=48):
    """First and last rows, both rows at every 256-row tile seam, and random rows."""
    seams = np.arange(tile, m, tile)
    rows = np.concatenate([np.arange(0, 4), seams - 1, seams, rng.choice(m, extra, replace=False),
                           np.arange(m - 4, m)])
    return np.unique(rows)


def test_block_1024_q4km_full_size(torch_cuda, qctx):
    b, s, p = 1, 4096, 256
    print("case: block 1024^2 Q4_K_M, hidden 4096, 32 heads, MLP 12288, 4096 tokens over 256", flush=True)
    w, x, mod, pe, kpre, vpre = make_case(4, CFG4, b, s, p, synth.Q4_K, synth.Q6_K)
    (got, (k, v)), (got_b, (kb, vb)) = run_modes(torch_cuda, qctx, CFG4, w, x, mod, pe, kpre, vpre, want_kv=True)
    assert np.isfinite(got).all() and np.isfinite(got_b).all()
    # the candle mode against the candle-mode oracle on every output row
    ref, kr, vr = O.block_forward(CFG4, w, x, mod, pe, kpre, vpre, mode=O.CANDLE)
    g2, r2 = got.reshape(s, -1), ref.reshape(s, -1)
    row_cos = np.sum(g2.astype(np.float64) * r2, 1) / np.sqrt(np.sum(np.square(g2, dtype=np.float64), 1) *
                                                            np.sum(np.square(r2, dtype=np.float64), 1))
    c, m = cos_sim(got, ref), max_abs_rel(got, ref)
    print(f"all rows: cos {c:.7f} mar {m:.2e}; lowest row cosine {row_cos.min():.7f}", flush=True)
    assert c >= 0.9999 and m <= 2e-2 and row_cos.min() >= 0.9999
    kv_close(k, kr)
    kv_close(v, vr)
    # sampled rows of both modes against both oracle modes, every K / V of the bf16 mode
    rows = sampled_rows(np.random.default_rng(40), s)
    ref_e, kre, vre = O.block_forward_rows(CFG4, w, x, mod, pe, rows, kpre, vpre, mode=O.EXACT)
    check_block(g2[rows], got_b.reshape(s, -1)[rows], r2[rows], ref_e, x.reshape(s, -1)[rows])
    kv_close(kb, kre)
    kv_close(vb, vre)


@pytest.mark.parametrize("attn_type,down_type,b,s", [(synth.Q8_0, synth.Q8_0, 1, 4352),
                                                     (synth.Q4_K, synth.Q6_K, 1, 4352),
                                                     (synth.Q8_0, synth.Q8_0, 2, 2176),
                                                     (synth.Q4_K, synth.Q6_K, 1, 4160),
                                                     (synth.Q8_0, synth.Q8_0, 1, 4102),
                                                     (synth.Q4_K, synth.Q6_K, 2, 2050)])
def test_block_4352_tokens_tail_rows(torch_cuda, qctx, attn_type, down_type, b, s):
    """4352 token rows at hidden 4096 (17 rows of 256x256 tiles): q/k/v makes
    816 tiles and out and down 272 for 256 CUs, so their last 256 token rows
    run as a 256-token product of their own (the 128x128 or split path; the
    gated residual on rows shifted by 4096, the q/k/v outputs, V^T and RoPE rows
    shifted to the tail's sequence and position: sequence 0 from position 4096,
    or with two sequences of 2176 tokens sequence 1 from position 1920), the
    rest as whole rounds; with 4160 tokens the last 64 rows take the short-M
    kernels (the gated residual and the f32 hidden state with its rows pass;
    q/k/v keeps them; with 4102 tokens, a token count that is not a multiple of
    the LayerNorm's four rows per workgroup, its last workgroup repeats the last
    row; with two sequences of 2050 tokens a workgroup's four rows span the
    sequence boundary, so it loads the second modulation row midway). Sampled
    rows, the seam at 4096, up to 48 of the last rows and the rows around a
    sequence boundary, and every token's K and V, against the candle-mode
    oracle."""
    p = 64
    m = b * s
    print(f"case: block hidden 4096, {b} x {s} tokens over {p}, types {attn_type}/{down_type}", flush=True)
    w, x, mod, pe, kpre, vpre = make_case(6, CFG4, b, s, p, attn_type, down_type)
    got, (k, v) = run_block(torch_cuda, qctx, CFG4, w, x, mod, pe, kpre, vpre, want_kv=True)
    assert np.isfinite(got).all()
    rng = np.random.default_rng(41)
    seam = np.arange(s - 4, s + 4) if b > 1 else np.arange(0)
    rows = np.unique(np.concatenate([sampled_rows(rng, m), rng.choice(np.arange(4096, m), min(48, m - 4096), replace=False),
                                     seam]))
    ref, kr, vr = O.block_forward_rows(CFG4, w, x, mod, pe, rows, kpre, vpre, mode=O.CANDLE)
    g = got.reshape(m, -1)[rows]
    c, mr = cos_sim(g, ref), max_abs_rel(g, ref)
    print(f"sampled rows: cos {c:.7f} mar {mr:.2e}", flush=True)
    assert c >= 0.9999 and mr <= 2e-2
    kv_close(k, kr)
    kv_close(v, vr)


def _q4k_negated(rows):
    """Q4_K rows [n, bytes] holding the exact negation of the given ones: the f16
    d and dmin of every 144-byte block change sign (value = d sc q - dmin m)."""
    out = rows.copy().reshape(rows.shape[0], -1, 144)
    out[:, :, 1] ^= 0x80
    out[:, :, 3] ^= 0x80
    return out.reshape(rows.shape)


def _tied_gate_up(w, mlp):
    """gate_up whose hidden state repeats each block's first 64 columns with
    signs -, -, + at offsets 64, 128, 192: every 256-value block of every row
    holds its largest magnitude four times, in both 128-column halves and in
    both 64-column groups of each, the first occurrence at the lowest column
    (gate rows copied, up rows copied or negated; silu(g) (-u) = -(silu(g) u))."""
    t, data, rows, cols = w["gate_up"]
    d = np.asarray(data).reshape(rows, -1).copy()
    for b in range(mlp // 256):
        c = 256 * b
        for off, neg in ((64, True), (128, True), (192, False)):
            d[c + off:c + off + 64] = d[c:c + 64]
            up = d[mlp + c:mlp + c + 64]
            d[mlp + c + off:mlp + c + off + 64] = _q4k_negated(up) if neg else up
    w["gate_up"] = (t, d.reshape(-1), rows, cols)


@pytest.mark.parametrize("case", ["1024x1024", "ragged_ties"])
def test_hidden_rounding_in_gate_up_epilogue_bit_identical(torch_cuda, qctx, monkeypatch, case):
    """The candle-mode Q8_K rounding of the SwiGLU hidden state, done by the
    large-M gate_up kernel's epilogue (one workgroup per pair of 256-row tiles,
    the 256 hidden columns of a Q8_K block), against the same rounding as its
    own pass after the GEMM (QIMM_SEPARATE_ROUNDING=1): bit-identical block
    outputs. Cases: the 1024^2 Q4_K_M block (4096 tokens, MLP 12288: 16 token
    tiles x 48 tile pairs), and hidden 1024 / MLP 4096 at 1100 tokens (a last
    token tile of 76 rows) with every block's largest magnitude tied four times
    across both tiles and both wave groups, opposite signs included."""
    if case == "1024x1024":
        cfg, b, s, p = CFG4, 1, 4096, 256
    else:
        cfg, b, s, p = dict(hidden=1024, heads=8, head_dim=128, mlp=4096), 1, 1100, 64
    print(f"case: {case}, hidden {cfg['hidden']}, MLP {cfg['mlp']}, {s} tokens", flush=True)
    w, x, mod, pe, kpre, vpre = make_case(21, cfg, b, s, p, synth.Q4_K, synth.Q6_K)
    if case == "ragged_ties":
        _tied_gate_up(w, cfg["mlp"])
    fused, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    monkeypatch.setenv("QIMM_SEPARATE_ROUNDING", "1")
    separate, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    assert np.isfinite(fused).all()
    diff = np.count_nonzero(fused.view(np.uint32) != separate.view(np.uint32))
    print(f"outputs differing in any bit: {diff} of {fused.size}", flush=True)
    assert diff == 0


def _tied_heads(w, kpre, vpre, heads):
    """q, k of head 2j + 1 copied from head 2j, its v (weights and prefix values)
    negated: the attention outputs of the pair are exact negations of each
    other, so every query's largest magnitude over the pair's 256 output
    columns ties across the two heads with opposite signs."""
    for name, neg in (("to_q", False), ("to_k", False), ("to_v", True)):
        t, data, rows, cols = w[name]
        d = np.asarray(data).reshape(rows, -1).copy()
        for j in range(0, heads, 2):
            src = d[128 * j:128 * (j + 1)]
            d[128 * (j + 1):128 * (j + 2)] = _q4k_negated(src) if neg else src
        w[name] = (t, d.reshape(-1), rows, cols)
    kpre[:, 1::2] = kpre[:, 0::2]
    vpre[:, 1::2] = vpre[:, 0::2] ^ np.uint16(0x8000)


@pytest.mark.parametrize("case", ["heads_tied"])
def test_attention_q8k_pair_rounding_bit_identical(torch_cuda, qctx, monkeypatch, case):
    """The candle-mode Q8_K rounding of the attention output (to_out's input,
    256 values = two heads of a query), done by the paired cached-step attention
    kernel (one workgroup per head pair, the first head's f32 output through
    scratch), against the rows-quantizer pass (QIMM_SEPARATE_ROUNDING=1):
    bit-identical block outputs, with the pair's maxima tied across the two
    heads with opposite signs in every query (the first head must win). Hidden
    4096, 32 heads, 2048 tokens over 256: the 8-wave form. The 1024^2 case of
    the gate_up test above covers the untied full size."""
    cfg, b, s, p = dict(hidden=4096, heads=32, head_dim=128, mlp=4096), 1, 2048, 256
    w, x, mod, pe, kpre, vpre = make_case(23, cfg, b, s, p, synth.Q4_K, synth.Q6_K)
    _tied_heads(w, kpre, vpre, cfg["heads"])
    fused, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    monkeypatch.setenv("QIMM_SEPARATE_ROUNDING", "1")
    separate, _ = run_block(torch_cuda, qctx, cfg, w, x, mod, pe, kpre, vpre)
    assert np.isfinite(fused).all()
    diff = np.count_nonzero(fused.view(np.uint32) != separate.view(np.uint32))
    print(f"{case}: outputs differing in any bit: {diff} of {fused.size}", flush=True)
    assert diff == 0


def multi_ref_pe(text_len, cond, grid):
    """RoPE rows of the target over a joint layout of text, condition images and
    the target (EmbedNd::forward, src/rope.rs:104-211): positions run on past the
    condition images, so the target's frame index is text_len + the images' extents."""
    shapes = [(1, g, g) for g in cond] + [(1, grid, grid)]
    mask = [0] * text_len + [1] * (sum(g * g for g in cond) + grid * grid)
    return O.rope_table(shapes, mask)[-grid * grid:]


def test_multi_ref_attention_full_size(torch_cuda, qctx):
    """Batch 2, 32 heads, 4096 queries over an 8448-token cached prefix plus 4096
    own keys (12544 keys): sampled query rows of both batch entries against the
    oracle's exact (f64) attention on the same bf16 Q/K/V."""
    b, h, sq, p = 2, 32, 4096, 8448
    print("case: multi-reference attention B2 H32 4096 queries, 8448 + 4096 keys", flush=True)
    got, q, ko, vo, kp, vp = _attention_case(torch_cuda, qctx, b, h, sq, p, sq, seed=5)
    assert np.isfinite(got).all()
    rows = np.array([0, 1, 31, 32, 255, 256, 1777, 2048, 3333, 4094, 4095])
    want = O.attention(q[:, :, rows], ko, vo, kp, vp, mode=O.EXACT)
    g = got[:, :, rows]
    assert cos_sim(g, want) >= 0.9999 and max_abs_rel(g, want) <= 2e-2, (cos_sim(g, want), max_abs_rel(g, want))
    for bb in range(b):
        assert cos_sim(g[bb], want[bb]) >= 0.9999


def test_multi_ref_block_q8_0_full_size(torch_cuda, qctx):
    """One Q8_0 block of the multi-reference step, both CFG prompts batched: 2 x 4096
    target tokens, each prompt over its own 8448-token bf16 prefix cache. Every K / V
    of each mode against the matching oracle mode; the output on sampled rows of both
    prompts in both modes."""
    b, s, p = 2, 4096, 8448
    print("case: multi-reference block Q8_0, B2 x 4096 tokens over 8448-token prefixes", flush=True)
    rng = np.random.default_rng(55)
    w = synth.block_weights(55, CFG4["hidden"], CFG4["heads"], CFG4["mlp"], synth.Q8_0, synth.Q8_0)
    x = rng.standard_normal((b, s, CFG4["hidden"]), dtype=np.float32)
    mod = (rng.standard_normal((b, 1, 4 * CFG4["hidden"]), dtype=np.float32) * 0.5).astype(np.float32)
    pe = multi_ref_pe(256, [64, 64], 64)
    kpre = O.f32_to_bf16(rng.standard_normal((b, CFG4["heads"], p, 128), dtype=np.float32))
    vpre = O.f32_to_bf16(rng.standard_normal((b, CFG4["heads"], p, 128), dtype=np.float32))
    (got, (k, v)), (got_b, (kb, vb)) = run_modes(torch_cuda, qctx, CFG4, w, x, mod, pe, kpre, vpre, want_kv=True)
    assert np.isfinite(got).all() and np.isfinite(got_b).all()
    r0 = sampled_rows(np.random.default_rng(56), s, extra=24)
    rows = np.concatenate([r0, s + r0])
    xr = x.reshape(b * s, -1)[rows]
    ref, kr, vr = O.block_forward_rows(CFG4, w, x, mod, pe, rows, kpre, vpre, mode=O.CANDLE)
    kv_close(k, kr)
    kv_close(v, vr)
    ref_e, kre, vre = O.block_forward_rows(CFG4, w, x, mod, pe, rows, kpre, vpre, mode=O.EXACT)
    kv_close(kb, kre)
    kv_close(vb, vre)
    check_block(got.reshape(b * s, -1)[rows], got_b.reshape(b * s, -1)[rows], ref, ref_e, xr)


Q8_SETS = {"qkv": (12288, 4096), "out": (4096, 4096), "up": (16384, 4096), "down": (4096, 16384)}


@pytest.mark.parametrize("m", [4352, 256])
@pytest.mark.parametrize("name", list(Q8_SETS))
def test_q8_0_gemm_sets_sampled_rows(torch_cuda, qctx, name, m):
    """A [m x K] bf16 ~ N(0,1) times a Q8_0 weight set from N(0, 0.02) (the GGML
    rule d = amax/127), bf16 output: sampled rows (every tile seam, head and
    tail) against the oracle's exact and candle modes."""
    torch = torch_cuda
    n, k = Q8_SETS[name]
    print(f"case: Q8_0 {name} {n}x{k} at {m} tokens", flush=True)
    rng = np.random.default_rng(n + k + m)
    _, w, _, _ = synth.weight(rng, synth.Q8_0, n, k)
    W = qctx.upload(synth.Q8_0, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k), dtype=np.float32))
    y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), synth.BF16, stream(torch))
    got = host(y.float())
    W.free()
    assert np.isfinite(got).all()
    rows = sampled_rows(rng, m, tile=128 if m < 512 else 256, extra=16)
    for mode in (O.EXACT, O.CANDLE):
        want = O.qmatmul(synth.Q8_0, w, n, k, a[rows], mode)
        g = got[rows]
        assert cos_sim(g, want) >= 0.9999 and max_abs_rel(g, want) <= 2e-2, (mode, cos_sim(g, want),
                                                                            max_abs_rel(g, want))
