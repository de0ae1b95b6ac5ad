"""GPU parity of candle's activation rounding (qimm_quantize_act, the quantize
step of QMatMul::forward, src/quantized_transformer.rs:19-29 -> candle-core
0.11 BlockQ8K / BlockQ8_0::from_float), through the C ABI.

Bars: the bf16 operands bf16(d * q) are bit-identical to the oracle's
(oq_quant_act_bf16) on the same f32 rows, including all-zero blocks, ties of
the largest magnitude with opposite signs and rows of mixed scales. A matmul
fed with them (qimm_quantize_act then qimm_qmatmul, the two halves of
QMatMul::forward) agrees with the oracle's candle mode (int8 codes, integer
dot products) to cosine >= 0.99999 and max|a-b|/max|b| <= 5e-3: the codes are
the same, only the bf16 rounding of d * q and of the weights remains.
"""
import numpy as np
import pytest

import oracle as O
import synth
from gpu_util import cos_sim, dev, host, max_abs_rel, stream
from test_oracle_act_quant import near_half_rows

pytestmark = pytest.mark.gpu


def _rows(seed, m, k):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * np.exp(rng.standard_normal((m, 1)))).astype(np.float32)
    x[0, :256] = 0.0
    if m > 1 and k >= 256:
        x[1, 5], x[1, 77] = -7.0, 7.0
        x[1, 130], x[1, 131] = 2.5, -2.5
    return x


def _quant_gpu(torch, qctx, wt, x, ldx=None):
    m, k = x.shape
    ldx = ldx or k
    xp = np.zeros((m, ldx), np.float32)
    xp[:, :k] = x
    xd = dev(torch, xp)
    out = torch.empty((m, k), dtype=torch.int16, device="cuda")
    qctx.quantize_act(wt, xd.data_ptr(), m, k, out.data_ptr(), ldx=ldx, ldo=k, stream=stream(torch))
    return host(out).view(np.uint16)


@pytest.mark.parametrize("wt,m,k", [(synth.Q4_K, 3, 256), (synth.Q4_K, 37, 4096), (synth.Q6_K, 5, 12288),
                                    (synth.Q8_0, 4, 32), (synth.Q8_0, 9, 96), (synth.Q8_0, 33, 4096),
                                    (synth.Q8_0, 2, 16384)])
def test_quantize_act_bit_exact(torch_cuda, qctx, wt, m, k):
    x = _rows(m * 7 + k, m, k)
    got = _quant_gpu(torch_cuda, qctx, wt, x)
    want = O.quant_act_bf16(wt, x)
    assert np.array_equal(got, want), np.count_nonzero(got != want)


@pytest.mark.parametrize("wt", [synth.Q4_K, synth.Q8_0])
def test_quantize_act_products_near_a_half_bit_exact(torch_cuda, qctx, wt):
    """Blocks whose products v * s round to exactly a half in float32 without
    being one (near_half_rows: ~100 values per 64 Q8_K blocks where a fused
    v * s + c, the contraction HIP device code allows by default, truncates to
    another code): the kernels round the float32 product first, as candle does,
    bit-identical to the oracle."""
    x = near_half_rows(wt, 11, 64).reshape(-1, 1024)
    got = _quant_gpu(torch_cuda, qctx, wt, x)
    want = O.quant_act_bf16(wt, x)
    assert np.array_equal(got, want), np.count_nonzero(got != want)


def test_quantize_act_strided_rows(torch_cuda, qctx):
    x = _rows(3, 6, 512)
    got = _quant_gpu(torch_cuda, qctx, synth.Q4_K, x, ldx=768)
    assert np.array_equal(got, O.quant_act_bf16(synth.Q4_K, x))


def test_quantize_act_rejects_bad_calls(torch_cuda, qctx):
    import qimm
    x = torch_cuda.zeros((2, 256), dtype=torch_cuda.float32, device="cuda")
    o = torch_cuda.zeros((2, 256), dtype=torch_cuda.int16, device="cuda")
    for wt, k in ((synth.BF16, 256), (synth.Q4_K, 128), (synth.Q8_0, 48)):
        with pytest.raises(qimm.QimmError):
            qctx.quantize_act(wt, x.data_ptr(), 2, k, o.data_ptr())


@pytest.mark.parametrize("wt", [synth.Q8_0, synth.Q4_K, synth.Q6_K])
@pytest.mark.parametrize("m,n,k", [(8, 256, 4096), (64, 384, 4096), (200, 256, 1024), (600, 512, 2048)])
def test_qmatmul_on_rounded_rows_matches_candle_mode(torch_cuda, qctx, wt, m, n, k):
    torch = torch_cuda
    rng = np.random.default_rng(m + n + k + wt)
    _, w, _, _ = synth.weight(rng, wt, n, k)
    W = qctx.upload(wt, n, k, w.tobytes())
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd = dev(torch, x)
    xq = torch.empty((m, k), dtype=torch.bfloat16, device="cuda")
    qctx.quantize_act(wt, xd.data_ptr(), m, k, xq.data_ptr(), stream=stream(torch))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    qctx.qmatmul(W, xq.data_ptr(), m, k, y.data_ptr(), synth.F32, stream(torch))
    got = host(y)
    W.free()
    want = O.qmatmul(wt, w, n, k, x, O.CANDLE)
    c, r = cos_sim(got, want), max_abs_rel(got, want)
    print(f"cos {c:.8f} mar {r:.2e}", flush=True)
    assert c >= 0.99999 and r <= 5e-3, (c, r)
