"""Pins the oracle's scalar conversions and GGML block codecs.

Known-answer blocks are written byte by byte from the GGML block layouts, with
expected values derived by hand (see the comments); conversions are checked
against numpy's IEEE binary16 and torch's bfloat16, which are independent
implementations. The quantizers only generate test inputs; they are checked
for validity (round-trip error bounds), not for bit-equality with candle.
"""
import numpy as np
import pytest

import oracle as O
import synth


def f16(x):
    return int(np.float16(x).view(np.uint16))


# ---------------------------------------------------------------- conversions

def test_f16_to_f32_all_65536_codes_match_numpy():
    L = O.lib()
    codes = np.arange(65536, dtype=np.uint32)
    got = np.array([L.oq_f16_to_f32(int(c)) for c in codes], dtype=np.float32)
    want = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_round_to_nearest_even_matches_numpy():
    L = O.lib()
    rng = np.random.default_rng(1)
    # exponents spanning f16 subnormal, normal and overflow ranges, plus exact halfway cases
    vals = (rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 18, 20000)).astype(np.float32)
    halfway = (np.arange(1, 2000, dtype=np.float32) + 0.5) * np.float32(2.0 ** -24)  # subnormal ties
    ties = np.float32(1.0) + np.arange(0, 64, dtype=np.float32) * np.float32(2.0 ** -11)
    vals = np.concatenate([vals, halfway, -halfway, ties, [0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e-8, np.inf]]).astype(np.float32)
    got = np.array([L.oq_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_round_to_nearest_even_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(50000) * 2.0 ** rng.integers(-20, 20, 50000)).astype(np.float32)
    special = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x00000001, 0x80000000],
                       dtype=np.uint32).view(np.float32)
    x = np.concatenate([x, special])
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    # 0x3F808000 is a tie with an even low half -> stays 0x3F80; 0x3F818000 rounds up to 0x3F82
    assert got[-6] == 0x3F80 and got[-5] == 0x3F82


# ---------------------------------------------------------------- Q8_0

Q8_CODES = [-128, -127, -100, -64, -33, -1, 0, 1, 2, 3, 17, 31, 32, 33, 63, 64,
            65, 100, 126, 127, -2, -3, -4, -5, 5, 6, 7, 8, 9, 10, 11, 12]


def q8_block(d_bits, codes):
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8], np.uint8),
                           np.array(codes, np.int8).view(np.uint8)])


@pytest.mark.parametrize("d_bits,scale", [(0x3C00, 1.0), (0xB800, -0.5), (0x0001, 2.0 ** -24),
                                          (0x7BFF, 65504.0), (0x0000, 0.0)])
def test_q8_0_known_answers(d_bits, scale):
    out = O.dequantize(O.Q8_0, q8_block(d_bits, Q8_CODES), 32)
    want = np.array(Q8_CODES, dtype=np.float64) * scale
    assert np.array_equal(out.astype(np.float64), want)


# ---------------------------------------------------------------- Q4_K

# scales bytes for sc = [1, 2, 3, 4, 63, 17, 33, 48], m = [5, 6, 7, 8, 63, 16, 32, 49]:
#   bytes 0..3  = sc[j] | (sc[j+4] >> 4) << 6   -> 0xC1 0x42 0x83 0xC4
#   bytes 4..7  = m[j]  | (m[j+4] >> 4) << 6    -> 0xC5 0x46 0x87 0xC8
#   bytes 8..11 = (sc[j+4] & 15) | (m[j+4] & 15) << 4 -> 0xFF 0x01 0x01 0x10
Q4K_SCALES = [0xC1, 0x42, 0x83, 0xC4, 0xC5, 0x46, 0x87, 0xC8, 0xFF, 0x01, 0x01, 0x10]
# qs[i] = i. Value v of 64-chunk c: v < 32 -> low nibble of qs[32c+v] (sub-block 2c),
# else high nibble of qs[32c+v-32] (sub-block 2c+1). Expected d*sc*q - dmin*m with d = dmin = 1:
Q4K_SPOTS = {0: -5, 1: -4, 31: 10, 32: -6, 63: -4, 64: -7, 79: 38, 96: 0, 128: -63, 129: 0,
             143: 882, 160: 52, 191: 69, 192: -32, 223: 463, 224: 239, 255: 287}


def q4k_block(d_bits, dmin_bits):
    return np.concatenate([np.array([d_bits & 0xFF, d_bits >> 8, dmin_bits & 0xFF, dmin_bits >> 8], np.uint8),
                           np.array(Q4K_SCALES, np.uint8), np.arange(128, dtype=np.uint8)])


def test_q4_k_known_answers():
    out = O.dequantize(O.Q4_K, q4k_block(0x3C00, 0x3C00), 256)
    for i, v in Q4K_SPOTS.items():
        assert out[i] == v, (i, out[i], v)
    # d = 0.5, dmin = 0.25: value 255 = 0.5*48*7 - 0.25*49 = 155.75
    out2 = O.dequantize(O.Q4_K, q4k_block(0x3800, 0x3400), 256)
    assert out2[255] == 155.75 and out2[0] == -1.25


# ---------------------------------------------------------------- Q6_K

Q6K_SCALES = [1, -1, 2, -2, 3, -3, 4, -4, 5, -5, 6, -6, 7, -7, 127, -128]
# ql[i] = i, qh[j] = j. Value idx in half h, w = idx % 128, r = w // 32, l = w % 32:
# low 4 bits from ql[64h + l + 32(r&1)] (low nibble if r < 2 else high), high 2 bits
# from qh[32h + l] >> 2r, q - 32, times scales[idx // 16] (hand-derived values):
Q6K_SPOTS = {0: -32, 5: -11, 16: 32, 35: -58, 45: 58, 70: -96, 100: -120, 127: 116, 128: -160,
             177: 186, 212: -147, 230: -3302, 240: 3200, 255: 3200}


def q6k_block(d_bits):
    return np.concatenate([np.arange(128, dtype=np.uint8), np.arange(64, dtype=np.uint8),
                           np.array(Q6K_SCALES, np.int8).view(np.uint8),
                           np.array([d_bits & 0xFF, d_bits >> 8], np.uint8)])


def test_q6_k_known_answers():
    out = O.dequantize(O.Q6_K, q6k_block(0x3C00), 256)
    for i, v in Q6K_SPOTS.items():
        assert out[i] == v, (i, out[i], v)
    out2 = O.dequantize(O.Q6_K, q6k_block(0x3800), 256)
    assert out2[230] == -1651.0


# ---------------------------------------------------------------- round trips

@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K])
def test_quantize_roundtrip_error_is_bounded(t):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(256 * 64) * 0.02).astype(np.float32)
    q = O.quantize(t, x)
    assert q.size == O.row_bytes(t, x.size)
    y = O.dequantize(t, q, x.size)
    rel = np.sqrt(np.mean((y - x) ** 2)) / np.sqrt(np.mean(x ** 2))
    assert rel < {O.Q8_0: 0.01, O.Q6_K: 0.03, O.Q4_K: 0.12}[t], rel


def test_q8_0_roundtrip_within_half_step():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(32 * 100).astype(np.float32)
    q = O.quantize(O.Q8_0, x).reshape(-1, 34)
    d = q[:, :2].copy().view(np.float16).astype(np.float32)[:, 0]
    y = O.dequantize(O.Q8_0, q.reshape(-1), x.size).reshape(-1, 32)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    # q = round(x * 127 / amax); y = q * f16(amax / 127)
    bound = d * 0.5 + 127 * np.abs(d - amax / 127) + 1e-7
    assert np.all(np.abs(y - x.reshape(-1, 32)) <= bound[:, None])


def test_q8_k_lossless_on_grid_values():
    # max-magnitude element -128*s makes iscale = 1/s: integer multiples of s are exact
    rng = np.random.default_rng(5)
    s = np.float32(2.0 ** -6)
    k = rng.integers(-127, 128, 256).astype(np.float32)
    k[17] = -128
    x = (k * s).astype(np.float32)
    y = O.dequantize(O.Q8_K, O.quantize(O.Q8_K, x), 256)
    assert np.array_equal(x, y)


@pytest.mark.parametrize("t", [synth.Q8_0, synth.Q4_K, synth.Q6_K])
def test_synth_quantizers_match_oracle_quantizers(t):
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((8, 512)) * 0.02).astype(np.float32)
    assert np.array_equal(synth.quantize(t, x), O.quantize(t, x))


def test_row_bytes():
    assert O.row_bytes(O.Q8_0, 4096) == 4096 // 32 * 34
    assert O.row_bytes(O.Q4_K, 4096) == 16 * 144
    assert O.row_bytes(O.Q6_K, 12288) == 48 * 210
    assert O.row_bytes(O.Q4_K, 100) == -1
