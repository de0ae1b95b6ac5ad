"""GPU parity: exact dequantization, the dequant-GEMM and the joint attention,
through the C ABI, against the oracle on the same seeded inputs.

Bars: dequantization bit-exact. GEMM: against float64 products of the same
bf16 activations and the bf16-rounded dequantized weights the MFMA consumes,
error <= 2e-4 of sum|a||w| per output (accumulation order only); and against
the oracle's exact and candle modes, cosine >= 0.9999 and
max|a-b|/max|b| <= 2e-2. Attention: against the oracle on the same bf16
Q/K/V, cosine >= 0.9999 and max|a-b|/max|b| <= 2e-2.
"""
import numpy as np
import pytest

import oracle as O
import synth
from gpu_util import bf16_dev, cos_sim, dev, host, max_abs_rel, stream
from test_oracle_codecs import q4k_block, q6k_block, q8_block, Q8_CODES

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------- dequant

def _dequant_gpu(torch, qctx, t, data, n):
    src = dev(torch, np.asarray(data, dtype=np.uint8))
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    qctx.dequant(t, src.data_ptr(), n, out.data_ptr(), stream(torch))
    return host(out)


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K, O.F16, O.BF16, O.F32])
def test_dequant_bit_exact_random(torch_cuda, qctx, t):
    rng = np.random.default_rng(100 + t)
    n = 256 * 37
    x = (rng.standard_normal(n) * 0.02 * 2.0 ** rng.integers(-8, 8, n)).astype(np.float32)
    data = O.quantize(t, x)
    got = _dequant_gpu(torch_cuda, qctx, t, data, n)
    want = O.dequantize(t, data, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_bit_exact_known_answer_blocks(torch_cuda, qctx):
    blocks = {
        O.Q8_0: np.concatenate([q8_block(b, Q8_CODES) for b in (0x3C00, 0xB800, 0x0001, 0x7BFF, 0x03FF)]),
        O.Q4_K: np.concatenate([q4k_block(0x3C00, 0x3C00), q4k_block(0x3800, 0x3400), q4k_block(0x0001, 0x0401)]),
        O.Q6_K: np.concatenate([q6k_block(0x3C00), q6k_block(0x3800), q6k_block(0x0003)]),
    }
    for t, data in blocks.items():
        n = data.size // O.lib().oq_block_bytes(t) * O.lib().oq_block_size(t)
        got = _dequant_gpu(torch_cuda, qctx, t, data, n)
        want = O.dequantize(t, data, n)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), t


# ---------------------------------------------------------------- GEMM

def _gemm_case(torch, qctx, t, m, n, k, seed, out_type=synth.F32, std=0.02):
    rng = np.random.default_rng(seed)
    _, w, _, _ = synth.weight(rng, t, n, k, std)
    W = qctx.upload(t, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    if out_type == synth.F32:
        y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    else:
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), out_type, stream(torch))
    got = host(y.float())
    W.free()
    return got, a, w


@pytest.mark.parametrize("t", [synth.Q8_0, synth.Q4_K, synth.Q6_K, synth.BF16])
@pytest.mark.parametrize("m,n,k", [(1, 128, 256), (17, 256, 512),
                                   # M <= 64 with K % 256 == 0: split-K weight streaming (a short
                                   # chunk, a partial 16-token tile, chunks longer than six stages)
                                   (16, 384, 4096), (33, 256, 1024), (64, 128, 8192),
                                   (130, 384, 1024), (300, 128, 4096),
                                   (600, 512, 1024), (1024, 256, 768),
                                   # 256x256 kernels (more 128x128 tiles than two per CU): the
                                   # eight-wave kernel for the quantized formats, one super-block and
                                   # four (every Q6_K scale-pair and half position, negative scales);
                                   # bf16 weights take the four-wave kernel's direct global->LDS path
                                   (2304, 4096, 256), (2304, 4096, 1024)])
def test_qmatmul_matches_bf16_weight_products(torch_cuda, qctx, t, m, n, k):
    """Products of the bf16 activations and the weights each path multiplies:
    bf16-rounded dequantized weights on the MFMA dequant paths, the exact Q4_K
    weights on the code-product path (Q4_K, M <= 16, K % 1024 == 0)."""
    got, a, w = _gemm_case(torch_cuda, qctx, t, m, n, k, seed=m * 7 + n + k + t)
    Wd = O.dequantize(t, w, n * k).reshape(n, k)
    Wb = O.bf16_round(Wd).astype(np.float64)
    want = a.astype(np.float64) @ Wb.T
    scale = np.abs(a).astype(np.float64) @ np.abs(Wb).T
    if t == synth.Q4_K and m <= 16 and k % 1024 == 0:
        want = a.astype(np.float64) @ Wd.astype(np.float64).T
    assert np.all(np.abs(got - want) <= 2e-4 * scale + 1e-6)
    # against the oracle: exact weights (exact mode) and candle's int8 activations
    ye = O.qmatmul(t, w, n, k, a, O.EXACT)
    assert cos_sim(got, ye) >= 0.9999 and max_abs_rel(got, ye) <= 2e-2
    if t != synth.BF16:
        yc = O.qmatmul(t, w, n, k, a, O.CANDLE)
        assert cos_sim(got, yc) >= 0.9999 and max_abs_rel(got, yc) <= 2e-2


@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096),
                                   (1, 8192, 4096),     # a single token
                                   (7, 12288, 4096),
                                   (5, 4096, 8192),     # eight 1024-k chunks
                                   (3, 1152, 1024),     # one k chunk
                                   (2, 12416, 4096),    # a second item for a few waves only
                                   (33, 4096, 4096),    # three 16-token tiles of 64 (one padded)
                                   (24, 2048, 2048),    # two 16-token tiles
                                   (64, 6144, 4096)])   # four full token tiles
def test_qmatmul_q4k_short_m_one_launch(torch_cuda, qctx, m, n, k):
    """Q4_K at M <= 64 and K % 1024 == 0 takes the one-launch kernel. Up to 16
    tokens it multiplies the raw codes and applies the scales afterwards: the
    product of the bf16 activations and the exact (not bf16-rounded) Q4_K
    weights, up to f32 summation order. From 17 tokens each weight is decoded
    once to bf16 for every token tile: the product with the bf16-rounded
    weights."""
    got, a, w = _gemm_case(torch_cuda, qctx, synth.Q4_K, m, n, k, seed=m + n + k)
    Wd = O.dequantize(synth.Q4_K, w, n * k).reshape(n, k)
    if m > 16:
        Wd = O.bf16_round(Wd)
    Wd = Wd.astype(np.float64)
    want = a.astype(np.float64) @ Wd.T
    scale = np.abs(a).astype(np.float64) @ np.abs(Wd).T
    assert np.all(np.abs(got - want) <= 2e-5 * scale + 1e-6), np.max(np.abs(got - want) / (scale + 1e-9))
    ye = O.qmatmul(synth.Q4_K, w, n, k, a, O.EXACT)
    assert cos_sim(got, ye) >= 0.9999 and max_abs_rel(got, ye) <= 2e-2
    yc = O.qmatmul(synth.Q4_K, w, n, k, a, O.CANDLE)
    assert cos_sim(got, yc) >= 0.9999 and max_abs_rel(got, yc) <= 2e-2


def test_qmatmul_short_m_one_launch_repeats(torch_cuda, qctx):
    """The M <= 64 Q4_K / Q6_K / Q8_0 path adds its split-K partial sums in
    the same launch, counting arrivals per output unit in counters that every
    call leaves at zero: calls in a row over different shapes, token counts and
    weights give bit-identical results to a first call, and match the
    products of the bf16 activations and the (bf16-rounded for Q6_K, Q8_0 and
    Q4_K beyond 16 tokens, exact for Q4_K up to 16) weights."""
    torch = torch_cuda
    cases = [(synth.Q6_K, 16, 4096, 3072), (synth.Q4_K, 16, 2048, 4096), (synth.Q6_K, 5, 1024, 12288),
             (synth.Q4_K, 1, 3072, 2048), (synth.Q6_K, 64, 4096, 3072), (synth.Q4_K, 40, 2048, 4096),
             (synth.Q6_K, 17, 1024, 2048), (synth.Q8_0, 16, 4096, 4096), (synth.Q8_0, 64, 2048, 2048),
             (synth.Q8_0, 3, 1024, 16384), (synth.Q6_K, 16, 4096, 3072),
             # one workgroup per 16-row group over the whole K (128-256 groups)
             (synth.Q6_K, 13, 4096, 12288), (synth.Q4_K, 16, 4096, 4096), (synth.Q8_0, 5, 2048, 16384),
             (synth.Q6_K, 1, 2048, 2048), (synth.Q4_K, 7, 3072, 6144)]
    first = {}
    for i, (t, m, n, k) in enumerate(cases * 2):
        rng = np.random.default_rng(100 + i % len(cases))
        _, w, _, _ = synth.weight(rng, t, n, k)
        W = qctx.upload(t, n, k, w.tobytes())
        a_dev, a = bf16_dev(torch, rng.standard_normal((m, k)).astype(np.float32))
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), synth.BF16, stream(torch))
        got = host(y.float())
        W.free()
        key = i % len(cases)
        if key in first:
            assert np.array_equal(got, first[key]), cases[key]
            continue
        first[key] = got
        Wd = O.dequantize(t, w, n * k).reshape(n, k)
        if t != synth.Q4_K or m > 16:
            Wd = O.bf16_round(Wd)
        want = a.astype(np.float64) @ Wd.astype(np.float64).T
        scale = np.abs(a).astype(np.float64) @ np.abs(Wd).astype(np.float64).T
        # bf16 output: half an ulp of the result on top of the f32 sums
        assert np.all(np.abs(got - want) <= 2e-5 * scale + 4e-3 * np.abs(want) + 1e-6), cases[key]


@pytest.mark.parametrize("t,m,n,out", [(synth.Q4_K, 64, 24576, synth.BF16), (synth.Q4_K, 20, 16384, synth.F32),
                                       (synth.Q6_K, 33, 16384, synth.BF16), (synth.Q8_0, 64, 16384, synth.BF16),
                                       (synth.Q8_0, 50, 24576, synth.F32), (synth.Q6_K, 17, 24576, synth.F32)])
def test_qmatmul_short_m_whole_k_per_workgroup(torch_cuda, qctx, t, m, n, out):
    """17-64 tokens at K = 4096 with 4 or 6 groups of 16 weight rows per CU
    (N 16384 or 24576 on 256 CUs): each workgroup keeps its groups over the
    whole K, x passing through LDS in 512-wide pieces, and two waves per group
    add their sums in a fixed order. Against the f64 product of the bf16
    activations and the bf16-rounded weights; a second call is bit-identical."""
    torch = torch_cuda
    k = 4096
    rng = np.random.default_rng(m + n)
    _, w, _, _ = synth.weight(rng, t, n, k)
    W = qctx.upload(t, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    dt = torch.bfloat16 if out == synth.BF16 else torch.float32
    got = []
    for _ in range(2):
        y = torch.empty((m, n), dtype=dt, device="cuda")
        qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), out, stream(torch))
        got.append(host(y.float()))
    W.free()
    assert np.array_equal(got[0], got[1])
    Wd = O.bf16_round(O.dequantize(t, w, n * k).reshape(n, k)).astype(np.float64)
    want = a.astype(np.float64) @ Wd.T
    scale = np.abs(a).astype(np.float64) @ np.abs(Wd).T
    tol = 2e-5 * scale + 1e-6 + (4e-3 * np.abs(want) if out == synth.BF16 else 0)
    assert np.all(np.abs(got[0] - want) <= tol), np.max(np.abs(got[0] - want) / (scale + 1e-9))


@pytest.mark.parametrize("m", [64, 700])
def test_qmatmul_bf16_output(torch_cuda, qctx, m):
    got, a, w = _gemm_case(torch_cuda, qctx, synth.Q4_K, m, 256, 512, seed=5, out_type=synth.BF16)
    want = O.qmatmul(synth.Q4_K, w, 256, 512, a, O.EXACT)
    assert cos_sim(got, want) >= 0.9999 and max_abs_rel(got, want) <= 2e-2


def test_qmatmul_full_qkv_shape_sampled_rows(torch_cuda, qctx):
    """M=4352 tokens x fused QKV [12288 x 4096] in Q8_0; rows sampled for the oracle."""
    torch = torch_cuda
    m, n, k = 4352, 12288, 4096
    rng = np.random.default_rng(7)
    _, w, _, _ = synth.weight(rng, synth.Q8_0, n, k)
    W = qctx.upload(synth.Q8_0, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), synth.F32, stream(torch))
    got = host(y)
    rows = np.concatenate([np.arange(0, 8), rng.choice(m, 16, replace=False), np.arange(m - 8, m)])
    want = O.qmatmul(synth.Q8_0, w, n, k, a[rows], O.EXACT)
    assert cos_sim(got[rows], want) >= 0.9999 and max_abs_rel(got[rows], want) <= 2e-2
    assert np.isfinite(got).all()
    W.free()


@pytest.mark.parametrize("m,n,k,t,out", [(4352, 4096, 4096, synth.Q4_K, synth.BF16),   # tail: split 128x128
                                         (4136, 4096, 4096, synth.Q4_K, synth.F32),    # tail: 40-row streaming
                                         (4352, 4096, 2048, synth.Q8_0, synth.BF16)])
def test_qmatmul_large_m_tail_rows(torch_cuda, qctx, m, n, k, t, out):
    """Large-M products whose last 256x256 tile row would run as a nearly empty
    wave hand those rows to the shorter-M paths (plain outputs): sampled head
    rows and every tail row match the products of the bf16 activations and
    the weights each path multiplies (bf16-rounded, or exact on the Q4_K
    code-product path), and the seam rows are continuous."""
    torch = torch_cuda
    rng = np.random.default_rng(m + k + t)
    _, w, _, _ = synth.weight(rng, t, n, k)
    W = qctx.upload(t, n, k, w.tobytes())
    a_dev, a = bf16_dev(torch, rng.standard_normal((m, k)).astype(np.float32))
    y = torch.empty((m, n), dtype=torch.float32 if out == synth.F32 else torch.bfloat16, device="cuda")
    qctx.qmatmul(W, a_dev.data_ptr(), m, k, y.data_ptr(), out, stream(torch))
    got = host(y.float())
    W.free()
    rows = np.concatenate([np.arange(0, 8), rng.choice(4096, 24, replace=False), np.arange(4090, m)])
    Wd = O.dequantize(t, w, n * k).reshape(n, k).astype(np.float64)
    Wb = O.bf16_round(Wd.astype(np.float32)).astype(np.float64)
    ar = a[rows].astype(np.float64)
    want_b, want_e = ar @ Wb.T, ar @ Wd.T
    scale = np.abs(ar) @ np.abs(Wb).T
    tol = 2e-4 * scale + 1e-6 + (4e-3 * np.abs(want_e) if out == synth.BF16 else 0)
    err = np.minimum(np.abs(got[rows] - want_b), np.abs(got[rows] - want_e))
    assert np.all(err <= tol), (rows[np.argmax((err - tol).max(axis=1))], float((err / (scale + 1e-9)).max()))
    assert np.isfinite(got).all()


def test_qmatmul_rejects_bad_shapes(torch_cuda, qctx):
    import qimm
    rng = np.random.default_rng(8)
    _, w, _, _ = synth.weight(rng, synth.Q8_0, 96, 64)   # N not a multiple of 128
    W = qctx.upload(synth.Q8_0, 96, 64, w.tobytes())
    x = torch_cuda.zeros((4, 64), dtype=torch_cuda.bfloat16, device="cuda")
    y = torch_cuda.zeros((4, 96), dtype=torch_cuda.float32, device="cuda")
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        qctx.qmatmul(W, x.data_ptr(), 4, 64, y.data_ptr(), synth.F32)
    W.free()
    with pytest.raises(qimm.QimmError, match="QIMM_ERR_SHAPE"):
        qctx.upload(synth.Q4_K, 128, 100, b"\0" * 10)
    # the K-quant device layouts interleave 16-row groups
    with pytest.raises(qimm.QimmError, match="rows % 16"):
        qctx.upload(synth.Q6_K, 24, 256, b"\0" * (24 * 210))
    with pytest.raises(qimm.QimmError, match="rows % 16"):
        qctx.upload(synth.Q4_K, 24, 256, b"\0" * (24 * 144))


# ---------------------------------------------------------------- attention

def _attention_case(torch, qctx, b, h, sq, p, so, seed, qmul=1.0):
    rng = np.random.default_rng(seed)
    q_dev, q = bf16_dev(torch, (qmul * rng.standard_normal((b, h, sq, 128))).astype(np.float32))
    ko_dev, ko = bf16_dev(torch, rng.standard_normal((b, h, so, 128)).astype(np.float32))
    vo = O.bf16_round(rng.standard_normal((b, h, so, 128)).astype(np.float32))
    vt_dev, _ = bf16_dev(torch, np.ascontiguousarray(vo.transpose(0, 1, 3, 2)))
    kv = None
    kp = vp = None
    if p > 0:
        kp_dev, kp = bf16_dev(torch, rng.standard_normal((b, h, p, 128)).astype(np.float32))
        vp_dev, vp = bf16_dev(torch, rng.standard_normal((b, h, p, 128)).astype(np.float32))
        kv = qctx.kv_create(2, b, h, p)
        kv.store(1, kp_dev.data_ptr(), vp_dev.data_ptr(), stream(torch))
        # round trip through the cache layout
        k2 = torch.empty_like(kp_dev)
        v2 = torch.empty_like(vp_dev)
        kv.load(1, k2.data_ptr(), v2.data_ptr(), stream(torch))
        assert torch.equal(k2, kp_dev) and torch.equal(v2, vp_dev)
    out = torch.empty((b, sq, h * 128), dtype=torch.bfloat16, device="cuda")
    qctx.attention(q_dev.data_ptr(), b, h, sq, kv, 1, ko_dev.data_ptr(), vt_dev.data_ptr(), so, 128 ** -0.5,
                   out.data_ptr(), stream(torch))
    got = host(out.float()).reshape(b, sq, h, 128).transpose(0, 2, 1, 3)
    if kv is not None:
        kv.free()
    return got, q, ko, vo, kp, vp


@pytest.mark.parametrize("b,h,sq,p,so,qmul", [
    (1, 2, 128, 64, 128, 1.0),    # aligned
    (1, 2, 200, 70, 200, 1.0),    # ragged query tile, unaligned prefix (per-element V^T path)
    (2, 3, 64, 256, 96, 1.0),     # batch 2, prefix longer than own; own tail window slides back
    (1, 1, 33, 0, 45, 1.0),       # no prefix, odd lengths
    (1, 2, 16, 8, 8, 1.0),        # tiny: both segments shorter than one 64-key block
    (1, 2, 300, 40, 520, 1.0),    # short prefix (clamped rows), own tail of 8 keys
    (2, 4, 256, 0, 136, 1.0),     # no prefix, own tail window slides back
    (1, 1, 513, 24, 64, 1.0),     # one query past a 256-query tile
    (1, 2, 256, 64, 448, 4.0),    # large score range: the running maximum moves mid-row
])
def test_attention_matches_oracle(torch_cuda, qctx, b, h, sq, p, so, qmul):
    got, q, ko, vo, kp, vp = _attention_case(torch_cuda, qctx, b, h, sq, p, so, seed=b + h + sq + p + so,
                                             qmul=qmul)
    want = O.attention(q, ko, vo, kp, vp, mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999, cos_sim(got, want)
    assert max_abs_rel(got, want) <= 2e-2, max_abs_rel(got, want)


@pytest.mark.parametrize("sq,p,so", [
    (200, 64, 448),   # prefix shorter than a key block (clamped rows); own tail window slides back past two halves
    (136, 40, 520),   # short prefix; own last window keeps only its last 32-key half
    (256, 256, 96),   # own segment shorter than a block: halves past its end are skipped
    (160, 0, 200),    # no prefix; the second window slides back past its first half
])
def test_attention_eight_wave_form_ragged_segments(torch_cuda, qctx, sq, p, so):
    """Batch 2 x 128 heads with 129-256 queries: 256 workgroups of 8 waves fill
    the CUs, so these ragged and short segments run through the 8-wave fast
    kernel (the small cases above take the 4-wave form)."""
    got, q, ko, vo, kp, vp = _attention_case(torch_cuda, qctx, 2, 128, sq, p, so, seed=sq + p + so)
    want = O.attention(q, ko, vo, kp, vp, mode=O.EXACT)
    assert cos_sim(got, want) >= 0.9999, cos_sim(got, want)
    assert max_abs_rel(got, want) <= 2e-2, max_abs_rel(got, want)


@pytest.mark.parametrize("sq", [4096, 2304])
def test_attention_config2_shape_sampled_rows(torch_cuda, qctx, sq):
    """B1 H32, sq image queries over 256 prefix + sq own keys; sampled query rows.
    4096 queries take the 8-wave fast kernel, 2304 the 4-wave one (two
    workgroups per CU)."""
    torch = torch_cuda
    b, h, p = 1, 32, 256
    got, q, ko, vo, kp, vp = _attention_case(torch, qctx, b, h, sq, p, sq, seed=2)
    rows = np.array([0, 1, 127, 128, 1000, 2047, 2175, sq - 2, sq - 1])
    want = O.attention(q[:, :, rows], ko, vo, kp, vp, mode=O.EXACT)
    g = got[:, :, rows]
    assert cos_sim(g, want) >= 0.9999 and max_abs_rel(g, want) <= 2e-2
    assert np.isfinite(got).all()


def test_qk_norm_rope_matches_oracle(torch_cuda, qctx):
    torch = torch_cuda
    rng = np.random.default_rng(9)
    b, s, h = 2, 40, 3
    x = rng.standard_normal((b, s, h, 128)).astype(np.float32)
    w = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    pe = O.rope_table([(1, 5, 8)], [1] * s)
    out = torch.empty((b, h, s, 128), dtype=torch.bfloat16, device="cuda")
    x_d, w_d, pe_d = dev(torch, x), dev(torch, w), dev(torch, pe)
    qctx.qk_norm_rope(x_d.data_ptr(), b, s, h, w_d.data_ptr(), pe_d.data_ptr(), out.data_ptr(), stream(torch))
    got = host(out.float())
    want = O.apply_rope(O.rmsnorm(x, w).transpose(0, 2, 1, 3), pe)
    assert np.max(np.abs(got - want)) <= 2 ** -7 * np.abs(want).max()
    vt = torch.empty((b, h, 128, s), dtype=torch.bfloat16, device="cuda")
    qctx.v_transpose(x_d.data_ptr(), b, s, h, vt.data_ptr(), stream(torch))
    assert np.array_equal(host(vt.float()), O.bf16_round(x.transpose(0, 2, 3, 1)))
