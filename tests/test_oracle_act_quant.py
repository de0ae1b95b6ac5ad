"""Pins the oracle's activation rounding (oq_quant_act_bf16): candle's CPU
QMatMul::forward quantizes each f32 input row to the weight's vec-dot type
(src/quantized_transformer.rs:19-29 -> candle-core 0.11 quantized/k_quants.rs,
BlockQ8K::from_float for Q4_K / Q6_K weights, BlockQ8_0::from_float for Q8_0
weights), and the GPU feeds the quantized values d * q to its MFMAs as bf16.

Pinned by an independent numpy restatement written from candle's code (f32
scale arithmetic, first-index maximum, half-away-from-zero rounding, the f16
scale of Q8_0) with its own bf16 rounding of the exact product (integer
rounding of the float64 bit pattern, not frexp/rint as in the C code), and by
known-answer blocks derived by hand, each chosen so that a plausible mistake
(the last instead of the first maximum, round-half-even, no clamp at 127, the
f32 instead of the f16 scale, a double-rounded product) fails.
"""
import numpy as np

import oracle as O


def _round_away(v):
    """Rust f32::round (half away from zero) of float32 values, exactly (in f64)."""
    v = v.astype(np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def _bf16_of_f64(v):
    """bf16 bits of float64 values rounded once to nearest even, by integer
    rounding of the f64 bit pattern (45 dropped mantissa bits); normal range."""
    v = np.asarray(v, dtype=np.float64)
    bits = v.view(np.uint64)
    keep = bits >> np.uint64(45)
    rem = bits & np.uint64((1 << 45) - 1)
    half = np.uint64(1 << 44)
    up = (rem > half) | ((rem == half) & ((keep & np.uint64(1)) == 1))
    keep = keep + up.astype(np.uint64)
    r = (keep << np.uint64(45)).view(np.float64).astype(np.float32)
    r[v == 0] = 0.0
    return (r.view(np.uint32) >> 16).astype(np.uint16)


def numpy_q8_k(x):
    x = np.asarray(x, dtype=np.float32).reshape(-1, 256)
    out = np.empty(x.shape, dtype=np.uint16)
    for b, xs in enumerate(x):
        i = int(np.argmax(np.abs(xs)))          # first index of the largest magnitude
        if np.abs(xs[i]) == 0:
            out[b] = 0
            continue
        iscale = np.float32(-128.0) / xs[i]
        q = np.minimum(_round_away(iscale * xs), 127.0)
        d = np.float32(1.0) / iscale
        out[b] = _bf16_of_f64(np.float64(d) * q)
    return out.reshape(-1)


def numpy_q8_0(x):
    x = np.asarray(x, dtype=np.float32).reshape(-1, 32)
    out = np.empty(x.shape, dtype=np.uint16)
    for b, xs in enumerate(x):
        amax = np.max(np.abs(xs))
        d = amax / np.float32(127.0)
        inv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        q = _round_away(xs * inv)
        d16 = np.float64(np.float16(d))
        out[b] = _bf16_of_f64(d16 * q)
    return out.reshape(-1)


def _near_half(s, kmax, vmax):
    """float32 values v (|v| < vmax) whose product with the float32 scale s
    rounds to exactly k + 1/2 (|k| < kmax) in float32 while the exact product
    is not k + 1/2: where rounding the product first (candle) and a fused
    v * s + c (a contracted multiply-add) may truncate to different codes."""
    s = np.float32(s)
    t = np.concatenate([np.arange(kmax) + 0.5, -(np.arange(kmax) + 0.5)])
    bits = (t / np.float64(s)).astype(np.float32).view(np.int32)
    cand = np.concatenate([(bits + o).view(np.float32) for o in range(-4, 5)])
    tt = np.tile(t, 9)
    p64 = cand.astype(np.float64) * np.float64(s)  # exact: 24 x 24 bits
    ok = (p64.astype(np.float32) == tt.astype(np.float32)) & (p64 != tt) & (np.abs(cand) < vmax)
    return np.unique(cand[ok])


def near_half_rows(wtype, seed, nblocks):
    """Rows of activation blocks for the weight type's rounding (Q8_K: 256
    values, Q8_0: 32), each block's largest magnitude first, the rest values
    whose products with the block's scale lie within half an float32 ulp of a
    half (_near_half), padded with zeros: the inputs on which an FMA
    contraction of the kernels' rounding would differ from candle's."""
    rng = np.random.default_rng(seed)
    qk = 256 if wtype in (O.Q4_K, O.Q6_K) else 32
    blocks = []
    while len(blocks) < nblocks:
        big = np.float32(rng.uniform(0.3, 5.0) * (1 if rng.integers(2) else -1))
        if qk == 256:
            s = np.float32(-128.0) / big
            v = _near_half(s, 127, abs(big))
        else:
            d = np.float32(abs(big)) / np.float32(127.0)
            v = _near_half(np.float32(1.0) / d, 127, abs(big))
        if len(v) == 0:
            continue
        b = np.zeros(qk, np.float32)
        b[0] = big
        v = rng.permutation(v)[:qk - 1]
        b[1:1 + len(v)] = v
        blocks.append(b)
    return np.concatenate(blocks)


def _f32_nearest(q):
    """The float32 nearest to the rational q, ties to even (one rounding)."""
    from fractions import Fraction
    f = np.float32(float(q))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        e = abs(Fraction(float(c)) - q)
        if best is None or e < best[0] or (e == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (e, c)
    return best[1]


def test_rounding_of_products_near_a_half():
    """On rows built from products that round to a half in float32 but are not
    one (near_half_rows), the oracle's activation rounding equals the numpy
    restatement (the product rounded to float32, then rounded half away from
    zero), and the rows hold such values: for each, the exact product plus the
    kernels' 0.49999997, rounded once (a fused multiply-add), truncates to a
    different code than the twice-rounded form in at least some cases."""
    from fractions import Fraction
    for wt, qk, restated in ((O.Q4_K, 256, numpy_q8_k), (O.Q8_0, 32, numpy_q8_0)):
        x = near_half_rows(wt, 5, 24)
        assert np.array_equal(O.quant_act_bf16(wt, x.reshape(-1, qk)).reshape(-1), restated(x))
        differs = 0
        for b in x.reshape(-1, qk):
            if qk == 256:
                s = np.float32(-128.0) / b[0]
            else:
                s = np.float32(1.0) / (np.float32(abs(b[0])) / np.float32(127.0))
            for v in b[1:][b[1:] != 0]:
                p32 = np.float32(v * s)
                c = np.float32(np.copysign(np.float32(0.49999997), p32))
                twice = np.trunc(np.float32(p32 + c))
                once = np.trunc(_f32_nearest(Fraction(float(v)) * Fraction(float(s)) + Fraction(float(c))))
                differs += int(once != twice)
        assert differs > 0, wt


def _rows(seed, m, k):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((m, k)) * np.exp(rng.standard_normal((m, 1)))).astype(np.float32)
    x[0, :256] = 0.0                              # an all-zero block
    x[1, 5], x[1, 77] = -7.0, 7.0                 # equal magnitudes, opposite signs: the first wins
    x[1, 100], x[1, 101] = 3.5, -3.5
    return x


def test_q8_k_rounding_matches_numpy_restatement():
    x = _rows(1, 6, 1024)
    for wt in (O.Q4_K, O.Q6_K):
        got = O.quant_act_bf16(wt, x)
        assert np.array_equal(got.reshape(-1), numpy_q8_k(x))


def test_q8_0_rounding_matches_numpy_restatement():
    x = _rows(2, 6, 1024)
    got = O.quant_act_bf16(O.Q8_0, x)
    assert np.array_equal(got.reshape(-1), numpy_q8_0(x))


def _val(b):
    """The f32 value of bf16 bits b."""
    return float(np.array([int(b) << 16], dtype=np.uint32).view(np.float32)[0])


def test_q8_k_known_answers():
    x = np.zeros(256, dtype=np.float32)
    x[3], x[10] = -2.0, 2.0        # first maximum -2: iscale 64, d 1/64; x[10] -> 128 -> clamped 127
    x[20], x[21] = 0.5, -0.0078125  # 0.5 * 64 = 32; -0.5 -> -1 (half away from zero; even gives 0)
    got = O.quant_act_bf16(O.Q4_K, x[None])[0]
    assert _val(got[3]) == -2.0
    assert _val(got[10]) == 127.0 / 64.0     # 1.984375, 8 significant bits: exact in bf16
    assert _val(got[20]) == 0.5
    assert _val(got[21]) == -1.0 / 64.0
    assert got[0] == 0
    # iscale = 1 (x_max = -128): 2.5 -> 3 and -2.5 -> -3 away from zero (2 and -2 to even)
    y = np.zeros(256, dtype=np.float32)
    y[0], y[1], y[2] = -128.0, 2.5, -2.5
    g = O.quant_act_bf16(O.Q6_K, y[None])[0]
    assert _val(g[0]) == -128.0 and _val(g[1]) == 3.0 and _val(g[2]) == -3.0
    # the all-zero block gives zeros (candle: d = 0, codes 0)
    assert np.all(O.quant_act_bf16(O.Q4_K, np.zeros((1, 256), np.float32)) == 0)


def test_q8_0_known_answers():
    # amax 127 * 2^-6: d = 2^-6 exactly in f16, q = x * 64
    x = np.zeros(32, dtype=np.float32)
    x[0], x[1], x[2] = 127.0 / 64.0, -1.0, 0.0234375   # 0.0234375 * 64 = 1.5 -> 2 (away from zero)
    got = O.quant_act_bf16(O.Q8_0, x[None])[0]
    assert _val(got[0]) == 127.0 / 64.0 and _val(got[1]) == -1.0 and _val(got[2]) == 2.0 / 64.0
    # amax 1: d = 1/127 rounds to the f16 2^-7 * (1 + 8/1024); x = 1 -> q = 127 ->
    # 127 * 0.00787353515625 = 0.99993896484375, whose nearest bf16 is 1.0;
    # x = 1/3 -> q = round(42.33) = 42 -> 0.3306884765625 -> bf16 0.330078125
    # (the f32 scale 1/127 would give 42/127 = 0.33070866 -> bf16 0.33203125)
    y = np.zeros(32, dtype=np.float32)
    y[0], y[1] = 1.0, np.float32(1.0 / 3.0)
    g = O.quant_act_bf16(O.Q8_0, y[None])[0]
    assert _val(g[0]) == 1.0
    assert _val(g[1]) == 0.330078125


def test_product_is_rounded_once():
    """d * q needs up to 32 significant bits, so its f32 rounding can land
    exactly halfway between two bf16 values and then round the wrong way. Over
    many random blocks the oracle's bits equal the once-rounded exact product
    (numpy restatement), and the twice-rounded variant (f32 product, then bf16)
    differs from it somewhere, so the test can tell the two apart."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((400, 256)).astype(np.float32)
    got = O.quant_act_bf16(O.Q4_K, x).reshape(-1)
    want = numpy_q8_k(x)
    assert np.array_equal(got, want)
    # the twice-rounded variant (f32 product, then bf16) differs somewhere
    twice = []
    for xs in x:
        i = int(np.argmax(np.abs(xs)))
        iscale = np.float32(-128.0) / xs[i]
        q = np.minimum(_round_away(iscale * xs), 127.0).astype(np.float32)
        d = np.float32(1.0) / iscale
        twice.append(O.f32_to_bf16((d * q).astype(np.float32)))
    assert not np.array_equal(np.concatenate(twice), want)


def _trunc_plus_below_half(x):
    """The kernels' round-half-away form (round_half_away in device_common.h):
    trunc(x + copysign(0.49999997f, x)), the sum rounded once in float32."""
    c = np.copysign(np.float32(0.49999997), x).astype(np.float32)
    return np.trunc((x + c).astype(np.float32))


def test_round_half_away_three_instruction_form_exhaustive():
    """trunc(x + copysign(largest float below 1/2, x)) equals half-away-from-zero
    rounding on every float32 with 2^-3 <= |x| < 2^8 (the |v s| <= 128 range of
    the activation codes; below 2^-3 both give 0), both signs: including the
    exact halves, the float just below each half, and 0.49999997 itself, where
    x + 0.5 would round up to 1."""
    lo = np.float32(2.0 ** -3).view(np.uint32)
    hi = np.float32(2.0 ** 8).view(np.uint32)
    step = 1 << 24
    for start in range(int(lo), int(hi), step):
        x = np.arange(start, min(start + step, int(hi)), dtype=np.uint32).view(np.float32)
        for v in (x, -x):
            got = _trunc_plus_below_half(v)
            want = _round_away(v)
            assert np.array_equal(got, want), v[np.nonzero(got != want)[0][:4]]
    small = np.array([0.0, 2.0 ** -30, 0.1249999, 0.25, 0.49999997], dtype=np.float32)
    assert np.array_equal(_trunc_plus_below_half(small), _round_away(small))
    assert np.array_equal(_trunc_plus_below_half(-small), _round_away(-small))


def test_product_for_bf16_form():
    """The kernels' bf16 operand of d * q (product_for_bf16 then round to
    nearest even): p = fma(d, q, +0) in float32, moved one ulp toward the exact
    product when p sits exactly halfway between two bf16 values with a nonzero
    error. Against the exact product's rounding (_bf16_of_f64) for random scales
    d and every code q in [-128, 127], plus scales chosen so that d * q lands
    exactly on a bf16 halfway point after its f32 rounding (the nudge in both
    directions) and q = 0 (+0 whatever d's sign)."""
    rng = np.random.default_rng(77)
    d = (rng.standard_normal(4096) * 10.0 ** rng.uniform(-6, 1, 4096)).astype(np.float32)
    # scales whose products with small codes round to bf16 halfway points:
    # an 8-bit significand plus the halfway bit, then one f32 ulp either way
    mid = ((rng.integers(128, 256, 2048) * 2 + 1) * 2.0 ** rng.integers(-20, 0, 2048)).astype(np.float32)
    for k in (3, 5, 7, 9, 11):
        t = (mid.astype(np.float64) / k).astype(np.float32)
        d = np.concatenate([d, t, np.nextafter(t, np.float32(0)), np.nextafter(t, np.float32(1e9)), -t])
    q = np.arange(-128, 128, dtype=np.float32)
    D, Q = np.meshgrid(d, q, indexing="ij")
    D, Q = D.ravel(), Q.ravel()
    exact = D.astype(np.float64) * Q.astype(np.float64)
    p = (exact + 0.0).astype(np.float32)  # f32 rounding of the exact product
    p[Q == 0] = np.float32(0.0)
    b = p.view(np.uint32).copy()
    e = exact - p.astype(np.float64)
    tie = ((b & 0xFFFF) == 0x8000) & (e != 0)
    same = (np.sign(e) == np.sign(p.astype(np.float64)))
    b[tie & same] += 1
    b[tie & ~same] -= 1
    pn = b.view(np.float32)
    r = pn.view(np.uint32)
    got = ((r + 0x7FFF + ((r >> 16) & 1)) >> 16).astype(np.uint16)
    want = _bf16_of_f64(exact)
    assert tie.sum() > 1000  # the halfway case is exercised
    assert np.array_equal(got, want)
    assert np.all(got[Q == 0] == 0)
