"""Order pins of the CPU oracle's f32 reductions -- CPU only.

Token identity with Camelid rests on the oracle folding every f32 sum in the reference's
order.  Each test below feeds an input whose correct result is worked out by hand from the
cited source order (in the comments, with exact binary values), and also evaluates the
plausible wrong variants -- reversed or pairwise order, a fused multiply-add where the source
rounds twice (or the reverse), a reassociated product -- step by step, asserting that every
variant gives different bits.  A reassociation, an OpenMP reduction or a contracted FMA in the
oracle therefore fails here, whatever the float64 bounds of test_oracle_pins.py allow.

Which order is "the CPU path" (Linux x86-64, the GPU box's host):
  - Q8_0 row fold           inference.rs:20434-20442 (sum += (float(dot) * w_d) * x_d, block order)
  - RMSNorm sum of squares  tensor/mod.rs:2083-2091 (ss += x * x, sequential)
  - attention score dot     tensor/mod.rs:2632-2648 dot_product (sequential, products rounded): the
                            Linux cache is KvDtype::F32 (kv_cache.rs:199-214) and the blocked
                            FMA lane is Windows-only (inference.rs:23932-23938)
  - softmax sum, AV         inference.rs:23988-24016 (score_sum += e, sequential; out[d] +=
                            prob * v[d], position order, no FMA)
  - Q4_K row dot            refmath.rs:539 and :559 (two fused multiply-adds per superblock,
                            mins first), the CPU decode's Q4_K dot (inference.rs:17906-17965)
  - Q6_K row dot            inference.rs:19282-19285 (8 class chains, then Rust's f32 Sum: a
                            left fold from -0.0)
"""
from fractions import Fraction

import numpy as np

F = np.float32


def rn(x: Fraction) -> float:
    """Round an exact rational to the nearest f32 (ties to even); normal range only."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    ulp = Fraction(2) ** (e - 23)
    q, r = divmod(a, ulp)
    q = int(q)
    if r * 2 > ulp or (r * 2 == ulp and q % 2 == 1):
        q += 1
    return float(sign * q * ulp)


def fma32(a, b, c) -> F:
    """f32 fused multiply-add: one rounding of the exact a*b + c."""
    return F(rn(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))))


def fold(terms, start=F(0.0)) -> F:
    s = F(start)
    for t in terms:
        s = F(s + F(t))
    return s


def pairwise(terms) -> F:
    t = [F(x) for x in terms]
    while len(t) > 1:
        t = [F(t[i] + t[i + 1]) if i + 1 < len(t) else t[i] for i in range(0, len(t), 2)]
    return t[0]


def bits(x) -> int:
    return int(np.asarray(x, np.float32).view(np.uint32))


def f16_bits(x: float) -> int:
    return int(np.asarray([x], np.float16).view(np.uint16)[0])


# ------------------------------------------------------------------ Q8_0 row fold
def _q8_row(dots, wds):
    """A Q8_0 wire row whose block b has weight scale wds[b] (f16) and a single nonzero quant
    dots[b] at position 0 (the activation has quant 1 at each block's position 0)."""
    row = np.zeros((len(dots), 34), np.uint8)
    for b, (dot, wd) in enumerate(zip(dots, wds)):
        row[b, :2] = np.frombuffer(np.uint16(f16_bits(wd)).tobytes(), np.uint8)
        row[b, 2] = np.uint8(np.int8(dot).view(np.uint8))
    return row.ravel()


def test_q8_0_row_fold_order_fma_and_association(orc):
    """inference.rs:20434-20442: term_b = (float(dot_b) * w_d) * x_d, two roundings, added in
    block order.  Six blocks; activation scales x_d = [1+2^-14, 1+2^-14, 1, 2^-12, 2^-12, 2^-12].
      row 0: dots (-1, +1), w_d = 1+2^-10: each term rounds (1+2^-10)(1+2^-14) = 1 + 2^-10 +
             2^-14 + 2^-24 to the even 1 + 2^-10 + 2^-14, so the two terms cancel: result 0.
             Fusing the second multiply into the add leaves the exact rounding error 2^-24.
      row 1: terms 1, 2^-24, 2^-24, 2^-24 (blocks 2..5): each 1 + 2^-24 is a tie that rounds
             to the even 1: result exactly 1.  Reversed or pairwise, the small terms combine
             first and survive.
      row 2: dot 3, w_d = 1+2^-10: 3(1+2^-10) = 3 + 3*2^-10 exactly, times (1+2^-14) =
             3 + 3*2^-10 + 3*2^-14 + 3*2^-24, rounded at ulp 2^-22 (0.75 ulp up): result
             3 + 3*2^-10 + 3*2^-14 + 2^-22.  float(dot) * (w_d * x_d) rounds w_d * x_d first."""
    a = 1 + 2 ** -10
    xs = np.array([1 + 2 ** -14, 1 + 2 ** -14, 1, 2 ** -12, 2 ** -12, 2 ** -12], np.float32)
    xq = np.zeros(6 * 32, np.int8)
    xq[::32] = 1
    rows = [_q8_row([-1, 1, 0, 0, 0, 0], [a, a, 1, 1, 1, 1]),
            _q8_row([0, 0, 1, 1, 1, 1], [1, 1, 1, 2 ** -12, 2 ** -12, 2 ** -12]),
            _q8_row([3, 0, 0, 0, 0, 0], [a, 1, 1, 1, 1, 1])]
    got = orc.q8_0_gemv(np.concatenate(rows), 3, 6 * 32, xs, xq)
    want = [0.0, 1.0, 3 + 3 * 2 ** -10 + 3 * 2 ** -14 + 2 ** -22]
    assert [bits(g) for g in got] == [bits(w) for w in want]
    # the wrong variants give other bits
    t_row0 = [F(F(F(-1) * F(a)) * xs[0]), F(F(F(1) * F(a)) * xs[1])]
    assert fold(t_row0) == 0.0
    fused = F(0.0)
    for dot, xd in ((-1, xs[0]), (1, xs[1])):
        fused = fma32(F(F(dot) * F(a)), xd, fused)
    assert bits(fused) == bits(2 ** -24) != bits(want[0])
    t_row1 = [F(1), F(2 ** -24), F(2 ** -24), F(2 ** -24)]
    assert bits(fold(t_row1)) == bits(want[1])
    assert bits(fold(t_row1[::-1])) != bits(want[1]) and bits(pairwise(t_row1)) != bits(want[1])
    reassoc = F(F(3) * F(F(a) * xs[0]))
    assert bits(reassoc) == bits(3 + 3 * 2 ** -10 + 3 * 2 ** -14) != bits(want[2])


# ------------------------------------------------------------------ RMSNorm sum of squares
def _rms_with_sum(x, w, ss, eps):
    n = F(len(x))
    scale = F(1.0) / np.sqrt(F(F(ss) / n) + F(eps))
    return (x * F(scale)) * w


def test_rms_norm_sum_order(orc):
    """tensor/mod.rs:2083-2091: ss += x*x in index order.  x = [1, 2^-12 x 15]: the squares
    are 1 and 15 x 2^-24; every 1 + 2^-24 is a tie that rounds to the even 1, so ss = 1,
    ms = 1/16, scale = 1/sqrt(1/16) = 4 and y = [4, 2^-10 x 15] exactly (w = 1, eps = 0).
    Reversed, the small squares sum to 15 * 2^-24 first and 1 + 15 * 2^-24 rounds to 1 + 2^-20;
    pairwise, they survive as well: both change the scale."""
    x = np.array([1.0] + [2 ** -12] * 15, np.float32)
    w = np.ones(16, np.float32)
    y = orc.rms_norm(x, w, 0.0)
    assert [bits(v) for v in y] == [bits(4.0)] + [bits(2 ** -10)] * 15
    sq = [F(v * v) for v in x]
    assert fold(sq) == 1.0
    for ss in (fold(sq[::-1]), pairwise(sq)):
        assert ss != 1.0
        assert not np.array_equal(_rms_with_sum(x, w, ss, 0.0).view(np.uint32), y.view(np.uint32))


def test_rms_norm_square_is_rounded_before_the_add(orc):
    """tensor/mod.rs:2083-2091: ss += x*x rounds the square, then the sum (Rust never contracts
    to an FMA).  x = [2^-12, 1 + 2^-12]: (1+2^-12)^2 = 1 + 2^-11 + 2^-24 rounds (tie, even) to
    1 + 2^-11; 2^-24 + (1 + 2^-11) is again a tie and rounds to 1 + 2^-11: ss = 1 + 2^-11.
    A fused multiply-add would give 1 + 2^-11 + 2^-23 and another output."""
    x = np.array([2 ** -12, 1 + 2 ** -12], np.float32)
    w = np.ones(2, np.float32)
    y = orc.rms_norm(x, w, 0.0)
    ss = F(1 + 2 ** -11)
    assert fold([F(v * v) for v in x]) == ss
    assert np.array_equal(y.view(np.uint32), _rms_with_sum(x, w, ss, 0.0).view(np.uint32))
    fused = fma32(x[1], x[1], fma32(x[0], x[0], F(0)))
    assert bits(fused) == bits(1 + 2 ** -11 + 2 ** -23)
    assert not np.array_equal(_rms_with_sum(x, w, fused, 0.0).view(np.uint32), y.view(np.uint32))


# ------------------------------------------------------------------ attention
def _attend(orc, q, keys, values, hd):
    n = len(keys)
    kc = np.zeros((1, n, hd), np.float32)
    vc = np.zeros((1, n, hd), np.float32)
    kc[0, :, :] = keys
    vc[0, :, :] = values
    return orc.attention(np.asarray(q, np.float32), kc, vc, 1, 1, hd, n, n)


def _softmax_av(scores, values, sum_order=fold, av_order="seq"):
    m = max(scores)
    e = [F(orc_expf(F(s - m))) for s in scores]
    inv = F(F(1.0) / sum_order(e))
    probs = [F(x * inv) for x in e]
    out = []
    for d in range(values.shape[1]):
        terms = [F(p * F(values[i, d])) for i, p in enumerate(probs)]
        out.append(fold(terms) if av_order == "seq" else fold(terms[::-1]))
    return np.array(out, np.float32)


_ORC = None


def orc_expf(x):
    return _ORC.expf(np.array([x], np.float32))[0]


def test_attention_score_dot_order(orc):
    """tensor/mod.rs:2632-2648 dot_product: sum += q_d * k_d in index order.  hd = 64 (scale
    1/8), two positions: k_0 = q = [8, 2^-9, 2^-9, 2^-9, 0...], so the products are 64 and
    3 x 2^-18, each 64 + 2^-18 a tie to the even 64: score_0 = 64/8 = 8 exactly; k_1 = 0
    (score 0).  Then e = [1, expf(-8)], out = [1/(1 + e_1), e_1/(1 + e_1)] through the
    orthogonal V rows.  Reversed (64 + 3*2^-18 -> 64 + 2^-16) or pairwise (64 + 2^-17), score_0
    moves by 2^-19 and e_1 with it."""
    global _ORC
    _ORC = orc
    hd = 64
    q = np.zeros(hd, np.float32)
    q[:4] = [8, 2 ** -9, 2 ** -9, 2 ** -9]
    keys = np.stack([q, np.zeros(hd, np.float32)])
    values = np.zeros((2, hd), np.float32)
    values[0, 0] = values[1, 1] = 1.0
    got = _attend(orc, q, keys, values, hd)
    prods = [F(a * b) for a, b in zip(q[:4], q[:4])]
    assert fold(prods) == 64.0
    want = _softmax_av([F(F(64.0) * F(0.125)), F(0.0)], values)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for s0 in (fold(prods[::-1]), pairwise(prods)):
        assert s0 != 64.0
        wrong = _softmax_av([F(s0 * F(0.125)), F(0.0)], values)
        assert not np.array_equal(wrong.view(np.uint32), got.view(np.uint32))


def test_attention_score_dot_products_are_rounded(orc):
    """tensor/mod.rs:2632-2648: sum += q_d * k_d, each product rounded before the add (no FMA).
    hd = 64 (scale 1/8), A = 16 + 2^-8, q = [A, -A, 8, 0...], k_0 = [A, A, 8, 0...], k_1 = 0:
      A * A = 256 + 2^-3 + 2^-16, a tie at ulp 2^-15, to even -> 256.125; -A * A -> -256.125;
      0 + 256.125 - 256.125 + 64 = 64, score_0 = 8 exactly, as in the order test above.
    A fused multiply-add keeps the second product exact: fma(-A, A, 256.125) = -2^-16, then
    fma(8, 8, -2^-16) = 64 - 2^-16 (exact at ulp 2^-18): score_0 = 8 - 2^-19, which moves
    e_1 = expf(score_1 - score_0) by about 2^-19 relative, i.e. many ulps."""
    global _ORC
    _ORC = orc
    hd = 64
    a = F(16 + 2.0 ** -8)
    q = np.zeros(hd, np.float32)
    q[:3] = [a, -a, 8]
    k0 = np.zeros(hd, np.float32)
    k0[:3] = [a, a, 8]
    keys = np.stack([k0, np.zeros(hd, np.float32)])
    values = np.zeros((2, hd), np.float32)
    values[0, 0] = values[1, 1] = 1.0
    got = _attend(orc, q, keys, values, hd)
    prods = [F(x * y) for x, y in zip(q[:3], k0[:3])]
    assert [float(v) for v in prods] == [256.125, -256.125, 64.0] and fold(prods) == 64.0
    want = _softmax_av([F(F(64.0) * F(0.125)), F(0.0)], values)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    fused = F(0.0)
    for x, y in zip(q[:3], k0[:3]):
        fused = fma32(x, y, fused)
    assert float(fused) == 64 - 2.0 ** -16
    wrong = _softmax_av([F(fused * F(0.125)), F(0.0)], values)
    assert not np.array_equal(wrong.view(np.uint32), got.view(np.uint32))


def test_attention_softmax_sum_and_av_order(orc):
    """inference.rs:23988-24016: the softmax denominator and each output are sequential folds
    in position order.  Position 0 holds the maximum score; the 600 later positions have
    e_p = expf(-2a/8) < 2^-24 (a = 69.3), so 1 + e_p rounds back to 1 every step: the
    denominator is exactly 1, inv = 1, prob_0 = 1, prob_p = e_p.  V column 1 is 1 at position
    0 only, so out[1] = prob_0 = inv = 1; V column 0 is 1 everywhere, so out[0] = 1*1 + sum of
    e_p * 1 (each add again rounding back) = 1 exactly.  Summing the e_p first (reversed or
    pairwise) keeps their total (~1.8e-5): in the denominator that moves out[1], in the
    output sum out[0]."""
    global _ORC
    _ORC = orc
    hd, n = 64, 601
    q = np.zeros(hd, np.float32)
    q[0] = 69.3
    keys = np.zeros((n, hd), np.float32)
    keys[0, 0] = 1.0
    keys[1:, 0] = -1.0
    values = np.zeros((n, hd), np.float32)
    values[:, 0] = 1.0
    values[0, 1] = 1.0
    got = _attend(orc, q, keys, values, hd)
    assert got[0] == 1.0 and got[1] == 1.0 and np.all(got[2:] == 0.0)
    scores = [F(F(F(69.3) * F(k)) * F(0.125)) for k in keys[:, 0]]
    e_p = F(orc_expf(F(scores[1] - scores[0])))
    assert 0 < e_p < 2 ** -24 and e_p * 600 > 2 ** -23
    assert np.array_equal(_softmax_av(scores, values[:, :2]), [1.0, 1.0])
    assert _softmax_av(scores, values[:, :2], sum_order=lambda e: fold(e[::-1]))[1] != 1.0
    assert _softmax_av(scores, values[:, :2], sum_order=pairwise)[1] != 1.0
    assert _softmax_av(scores, values[:, :2], av_order="rev")[0] != 1.0


def test_attention_av_product_is_rounded_before_the_add(orc):
    """inference.rs:24008-24011: out[d] += prob * v[d], the product rounded before the add.
    q = 0 makes three equal scores: e = [1, 1, 1], denominator 3, p = RN(1/3) for every
    position.  With v[0] = [1, -(1+2^-10), 0]: out = p, then p + RN(-p(1+2^-10)), then + 0.
    p(1+2^-10) = 11184811 * 1025 * 2^-35 is inexact, so the sequential result is -(RN(p(1+2^-10))
    - p) while a fused multiply-add gives the exact -p * 2^-10."""
    hd = 64
    q = np.zeros(hd, np.float32)
    keys = np.zeros((3, hd), np.float32)
    values = np.zeros((3, hd), np.float32)
    values[:, 0] = [1.0, -(1 + 2 ** -10), 0.0]
    got = _attend(orc, q, keys, values, hd)
    p = F(F(1.0) / F(3.0))
    want = F(F(p * F(1.0)) + F(p * F(-(1 + 2 ** -10))))
    assert bits(got[0]) == bits(want)
    fused = fma32(p, F(-(1 + 2 ** -10)), F(p * F(1.0)))
    assert bits(fused) == bits(-float(p) * 2 ** -10) != bits(want)


# ------------------------------------------------------------------ Q4_K row dot
def _q4k_superblock(d_w, dmin_w, scales, mins, nib0):
    """A Q4_K superblock (144 bytes: f16 d, f16 dmin, 12 packed 6-bit scale/min bytes, 128
    nibble bytes) with sub-block scales/mins < 4 (packed as tensor/mod.rs:4776-4785 reads
    them: sub-block g < 4 -> scale byte g, min byte g + 4; sub-blocks 4..7 unused here) and,
    per sub-block g, the nibble nib0[g] at the sub-block's first value (all others 0)."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.uint16(f16_bits(d_w)).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.uint16(f16_bits(dmin_w)).tobytes(), np.uint8)
    for g in range(4):
        assert scales[g] < 64 and mins[g] < 64
        b[4 + g] = scales[g]
        b[8 + g] = mins[g]
    for g in range(8):
        j, hi = g // 2, g % 2
        b[16 + 32 * j] |= np.uint8(nib0[g] << (4 * hi))
    return b


def test_q4_k_dot_fma_chain(orc):
    """refmath.rs:503-561: per superblock sumf = fma(-dmin, prod, sumf), then sumf =
    fma(d, sumi, sumf), d = y.d * f16(d_w), dmin = y.d * f16(dmin_w).  One superblock with
    y.d = 1, d_w = 1 + 2^-10, dmin_w = 1; activation quants a = [113, 127, 127, 57, 0...] at
    the first value of sub-blocks 0..3; sub-block 0 has scale 29 and nibble 5, sub-blocks 1..3
    have mins 63, 63, 7.  So sumi = 5*113*29 = 16385 and prod = 127*63 + 127*63 + 57*7 = 16401.
    d * sumi = 16385 + 16385*2^-10 = 16401 + 2^-10 exactly (needs one fused rounding).
    mins first: sumf = -16401; then fma(d, 16385, -16401) = 2^-10 exactly.  Rounding d * sumi
    first (a tie at ulp 2^-9, to the even 16401) gives 0; so does the scales-first order."""
    sb = _q4k_superblock(1 + 2 ** -10, 1.0, [29, 0, 0, 0], [0, 63, 63, 7], [5, 0, 0, 0, 0, 0, 0, 0])
    yq = np.zeros(256, np.int8)
    yq[[0, 32, 64, 96]] = [113, 127, 127, 57]
    got = orc.kquant_gemv(1, sb, 1, 256, np.array([1.0], np.float32), yq)
    assert bits(got[0]) == bits(2 ** -10)
    d, dmin, S, M = F(1 + 2 ** -10), F(1.0), 16385, 16401
    assert fma32(d, F(S), fma32(-dmin, F(M), F(0))) == F(2 ** -10)
    unfused = F(F(F(0) + F(-dmin * F(M))) + F(d * F(S)))
    scales_first = fma32(-dmin, F(M), fma32(d, F(S), F(0)))
    assert bits(unfused) == bits(0.0) and bits(scales_first) == bits(0.0)


# ------------------------------------------------------------------ Q6_K row dot
def _q6k_superblock(a, scales, d_w):
    """A Q6_K superblock (210 bytes: ql[128], qh[64], i8 scales[16], f16 d) holding the signed
    6-bit weights a[256] in value order (the layout inference.rs:19256-19276 decodes)."""
    u = (np.asarray(a, np.int32) + 32).astype(np.uint8)
    assert np.all(u < 64)
    b = np.zeros(210, np.uint8)
    for n in range(2):
        ql, qh, w = 64 * n, 128 + 32 * n, 128 * n
        for l in range(32):
            b[ql + l] = (u[w + l] & 0xF) | ((u[w + l + 64] & 0xF) << 4)
            b[ql + l + 32] = (u[w + l + 32] & 0xF) | ((u[w + l + 96] & 0xF) << 4)
            b[qh + l] = (u[w + l] >> 4) | ((u[w + l + 32] >> 4) << 2) | ((u[w + l + 64] >> 4) << 4) | \
                ((u[w + l + 96] >> 4) << 6)
    b[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    b[208:210] = np.frombuffer(np.uint16(f16_bits(d_w)).tobytes(), np.uint8)
    return b


def test_q6_k_dot_class_chains_and_left_fold(orc):
    """inference.rs:19240-19295: sums[l] += (f16(d_w) * y.d) * aux[l] per superblock, l the
    position mod 8, then the left fold of sums[0..8].  Superblock 0 (d = 1) has aux = [1, 0..]:
    sums[0] = 1.  Superblock 1 (d = 2^-12 * 2^-12 = 2^-24) has aux = [0, 1 x 7]: sums[1..8] =
    2^-24.  The left fold -0 + 1 + 2^-24 + ... rounds every tie back to 1: result 1.  Pairwise
    or reversed, and the single-accumulator order (q6_k_dot_scalar: sumf += d * sum of aux),
    keep the small terms: 1 + 2^-23 * k."""
    a0 = np.zeros(256, np.int32)
    a0[0] = 1
    a1 = np.zeros(256, np.int32)
    a1[1:8] = 1
    scales = [1] + [0] * 15
    wire = np.concatenate([_q6k_superblock(a0, scales, 1.0), _q6k_superblock(a1, scales, 2 ** -12)])
    # the encoder round-trips through the fixture-pinned decode (d * scale * a)
    deq = orc.dequant_kquant(2, wire)
    assert deq[0] == 1.0 and np.all(deq[256 + 1:256 + 8] == 2 ** -12) and np.count_nonzero(deq) == 8
    yq = np.zeros(512, np.int8)
    yq[0] = 1
    yq[256 + 1:256 + 8] = 1
    yd = np.array([1.0, 2 ** -12], np.float32)
    got = orc.kquant_gemv(2, wire, 1, 512, yd, yq)
    assert bits(got[0]) == bits(1.0)
    sums = [F(1.0)] + [F(2 ** -24)] * 7
    assert fold(sums, F(-0.0)) == 1.0
    single = fold([F(F(1.0) * F(1)), F(F(2 ** -24) * F(7))])
    for wrong in (pairwise(sums), fold(sums[::-1]), single):
        assert bits(wrong) != bits(1.0)
