"""Known-answer pins of the CPU oracle's elementwise f32 expressions -- CPU only.

test_oracle_order_pins.py fixes the order of every f32 reduction; this file fixes the shape of
every other f32 expression the oracle restates: where the reference divides and where it
multiplies by a reciprocal, which product it rounds first, and where it rounds a product
before an add.  Each test feeds an input whose result under the cited reference expression is
worked out below as exact binary values (the literals are f32 bit patterns; each step's
rounding is recomputed with exact rationals so the derivation is checked, not just stated),
asserts the oracle returns those bits, and evaluates the plausible rewrites of the expression
step by step, asserting that each one gives different bits.  A rewrite of any of these
expressions in the oracle therefore fails here, while float64 tolerances would pass it.

Transcendental steps (expf, powf) enter through their correctly rounded values, computed here
in 60-digit decimal arithmetic; every input is chosen so that the exact value lies well inside
its f32 rounding interval (the distance is asserted), where glibc's expf (error < 0.502 ulp)
and powf (< 0.82 ulp, and the exact value within 0.29 ulp of the result here) cannot return
another float.  sqrt is IEEE-exact.

Reference expressions (Linux x86-64, the scalar CPU path):
  - SwiGLU            tensor/mod.rs:1957, :1963  (g / (1 + exp(-g))) * u
  - RMSNorm           tensor/mod.rs:2082, :2093  ms = ss / n; scale = 1 / sqrt(ms + eps);
                                                 out = (x * scale) * w   (left to right)
  - attention score   inference.rs:23969         dot_product(q, k) * scale, scale =
                      diagnostic_config.rs:302   1 / sqrt(hd as f32)
  - softmax           inference.rs:23999-24002   inv = 1 / sum; prob = e * inv
  - RoPE rotation     rope.rs:514-515            x0' = (x0 * c) - (x1 * s), x1' = (x0 * s) + (x1 * c),
                                                 every product rounded (Rust never contracts)
  - RoPE frequency    rope.rs:526-529            powf(base, -(i * 2.0) / rope_dim)
  - llama3 smoothing  rope.rs:687-711            ((1 - smooth) * f / factor) + (smooth * f)
  - Q8_0 quantize     inference.rs:16962-16968   unrounded = amax / 127; inv = 1 / unrounded;
                                                 q = round(x * inv)
  - Q8_K quantize     inference.rs:17584-17590   iscale = -127 / max; q = nearest_int(iscale * x);
                                                 d = 1 / iscale
"""
from decimal import Decimal, getcontext
from fractions import Fraction

import numpy as np

from test_oracle_order_pins import bits, fma32, rn

F = np.float32
getcontext().prec = 60


def h(s: str) -> F:
    """An f32 from its C99 hex literal (exactly representable by construction)."""
    v = float.fromhex(s)
    assert float(F(v)) == v
    return F(v)


def _ulp(x: float) -> Fraction:
    _, e = np.frexp(x)
    return Fraction(2) ** (int(e) - 24)


def correctly_rounded(exact: Decimal) -> tuple[F, float]:
    """(the f32 nearest to exact, exact's distance from it in ulps of that f32)."""
    r = rn(Fraction(exact))
    return F(r), float((Fraction(exact) - Fraction(r)) / _ulp(r))


def expf_cr(x) -> F:
    r, dist = correctly_rounded(Decimal(float(x)).exp())
    assert abs(dist) < 0.45, "input too close to a rounding boundary for a known answer"
    return r


def powf_cr(b, e) -> F:
    r, dist = correctly_rounded((Decimal(float(e)) * Decimal(float(b)).ln()).exp())
    assert abs(dist) < 0.3, "input too close to a rounding boundary for a known answer"
    return r


def sqrtf_cr(x) -> F:
    return correctly_rounded(Decimal(float(x)).sqrt())[0]


def q8_0_round(v: F) -> int:
    """Rust f32::round (half away from zero) then clamp to [-128, 127]."""
    r = np.sign(v) * np.floor(np.abs(np.float64(v)) + 0.5)
    return int(np.clip(r, -128, 127))


# ------------------------------------------------------------------ SwiGLU
def test_swiglu_divides_g_then_multiplies_u(orc):
    """tensor/mod.rs:1957/:1963: (g / (1 + exp(-g))) * u, g = 0.875 = 0x1.cp-1, u = 0.625.
      exp(-0.875) = 0.41686201967850839...  -> e = 0x1.aadde0p-2 (the exact value is 0.29 ulp
                                               above e)
      1 + e                                  = 0x1.6ab778p+0 (exact: e's last bit is 2^-21)
      g / (1 + e)  = 0.61786...              -> t = RN(...)
      t * u                                  -> 0x1.8b3d56p-2
    Dividing u first, g*(u/(1+e)), multiplying g*u first, or forming the sigmoid 1/(1+e) and
    multiplying, each rounds a different intermediate and lands on 0x1.8b3d58p-2."""
    g, u = F(0.875), F(0.625)
    e = expf_cr(-g)
    assert bits(e) == bits(h("0x1.aadde0p-2"))
    den = F(F(1) + e)
    assert bits(den) == bits(h("0x1.6ab778p+0"))
    want = h("0x1.8b3d56p-2")
    assert bits(F(F(g / den) * u)) == bits(want)
    got = orc.silu_mul(np.array([g], F), np.array([u], F))[0]
    assert bits(got) == bits(want)
    wrong = [F(g * F(u / den)), F(F(g * u) / den), F(F(F(F(1) / den) * g) * u)]
    assert all(bits(w) == bits(h("0x1.8b3d58p-2")) for w in wrong)


# ------------------------------------------------------------------ RMSNorm output
def test_rms_norm_scale_and_output_association(orc):
    """tensor/mod.rs:2082/:2093 with eps = 1e-5 (f32 0x1.4f8b58p-17) on a 5-value row:
      x = (3.75, 0, 0.375, -0.375, 3.25), w = (0.5625, 0.1875, 1.8125, 1.5, 0.1875)
      ss = 14.0625 + 0 + 0.140625 + 0.140625 + 10.5625 = 24.90625 (every step exact)
      ms = ss / 5                 -> 0x1.3ecccc0p+2 (4.98125 rounded)
      ms + eps                    -> 0x1.3eccf6p+2
      sqrt(ms + eps)              -> 0x1.1dae08p+1
      scale = 1 / sqrt(...)       -> 0x1.caceb0p-2
      out_0 = (3.75 * scale) * 0.5625 -> 0x1.e3e5fcp-1
    The rewrites give other bits: scale as sqrt(1 / (ms + eps)) = 0x1.caceaep-2, without eps
    0x1.caceccp-2, with ms = ss * (1 / n) 0x1.caceacp-2; out_0 as x * (scale * w) =
    0x1.e3e600p-1, as (x * w) * scale = 0x1.e3e5fep-1."""
    x = np.array([3.75, 0.0, 0.375, -0.375, 3.25], F)
    w = np.array([0.5625, 0.1875, 1.8125, 1.5, 0.1875], F)
    eps = F(1e-5)
    assert bits(eps) == bits(h("0x1.4f8b58p-17"))
    ss = F(0)
    for v in x:
        ss = F(ss + F(v * v))
    assert float(ss) == 24.90625
    ms = F(ss / F(5))
    assert bits(ms) == bits(h("0x1.3ecccc0p+2"))
    a = F(ms + eps)
    assert bits(a) == bits(h("0x1.3eccf6p+2"))
    assert bits(sqrtf_cr(a)) == bits(h("0x1.1dae08p+1"))
    scale = F(F(1) / sqrtf_cr(a))
    assert bits(scale) == bits(h("0x1.caceb0p-2"))
    want = [F(F(v * scale) * wv) for v, wv in zip(x, w)]
    assert bits(want[0]) == bits(h("0x1.e3e5fcp-1"))
    got = orc.rms_norm(x[None], w, float(eps))[0]
    assert [bits(g) for g in got] == [bits(v) for v in want]
    # the rewrites of the scale
    assert bits(sqrtf_cr(F(F(1) / a))) == bits(h("0x1.caceaep-2"))
    assert bits(F(F(1) / sqrtf_cr(ms))) == bits(h("0x1.caceccp-2"))
    assert bits(F(F(1) / sqrtf_cr(F(F(ss * F(F(1) / F(5))) + eps)))) == bits(h("0x1.caceacp-2"))
    # the rewrites of the output association
    assert bits(F(x[0] * F(scale * w[0]))) == bits(h("0x1.e3e600p-1"))
    assert bits(F(F(x[0] * w[0]) * scale)) == bits(h("0x1.e3e5fep-1"))


# ------------------------------------------------------------------ attention scale and softmax
def _attention(orc, hd, keys0, n_pos):
    """One head, q = e_0, key p = (t_p, 0, ...): score_p = t_p * scale; value p = e_p, so output
    dim d is exactly prob_d (every other product is +0 and adds nothing)."""
    q = np.zeros(hd, F)
    q[0] = 1
    kc = np.zeros((n_pos, hd), F)
    kc[:, 0] = keys0
    vc = np.zeros((n_pos, hd), F)
    vc[np.arange(n_pos), np.arange(n_pos)] = 1
    return orc.attention(q, kc, vc, 1, 1, hd, n_pos, n_pos).ravel()[:n_pos]


def test_attention_score_scale_is_a_reciprocal_product_at_hd_128(orc):
    """inference.rs:23969 score = dot * scale, diagnostic_config.rs:302 scale = 1 / sqrt(128f32):
      sqrt(128) -> 0x1.6a09e6p+3, scale = 1 / that -> 0x1.6a09e6p-4.
    Keys t = (5.671875, 6.671875):
      s_0 = 5.671875 * scale -> 0x1.00ae04p-1, s_1 -> 0x1.2def42p-1 (the max)
      exp(s_0 - s_1) = exp(-0x1.8fa4e0p-4...)   -> e_0 = 0x1.d4b000p-1 (exact value 0.10 ulp
                                                     above)
      sum = e_0 + 1, inv = 1 / sum, probs (e_0 * inv, inv) = (0x1.e96328p-2, 0x1.0b4e6ep-1).
    Dividing by sqrt(128) instead, s_0 = 5.671875 / 0x1.6a09e6p+3 -> 0x1.00ae06p-1, one ulp
    higher, which gives prob_0 = 0x1.e9632ap-2."""
    sq = sqrtf_cr(F(128))
    assert bits(sq) == bits(h("0x1.6a09e6p+3"))
    scale = F(F(1) / sq)
    assert bits(scale) == bits(h("0x1.6a09e6p-4"))
    t = [F(5.671875), F(6.671875)]
    s = [F(v * scale) for v in t]
    assert [bits(v) for v in s] == [bits(h("0x1.00ae04p-1")), bits(h("0x1.2def42p-1"))]
    e0 = expf_cr(F(s[0] - s[1]))
    assert bits(e0) == bits(h("0x1.d4b000p-1"))
    inv = F(F(1) / F(e0 + F(1)))
    want = [F(e0 * inv), inv]
    assert [bits(v) for v in want] == [bits(h("0x1.e96328p-2")), bits(h("0x1.0b4e6ep-1"))]
    got = _attention(orc, 128, t, 2)
    assert [bits(v) for v in got] == [bits(v) for v in want]
    # the rewrite: divide by sqrt(hd)
    sv = [F(v / sq) for v in t]
    assert bits(sv[0]) == bits(h("0x1.00ae06p-1")) and bits(sv[1]) == bits(s[1])
    ev = expf_cr(F(sv[0] - sv[1]))
    invv = F(F(1) / F(ev + F(1)))
    assert bits(F(ev * invv)) == bits(h("0x1.e9632ap-2")) != bits(want[0])


def test_attention_softmax_multiplies_by_the_reciprocal_sum(orc):
    """inference.rs:23999-24002: inv = 1 / sum, prob = e * inv.  hd = 4 (scale = 1/2 exactly),
    keys t = (5.5, -2.5, 3.25, -4.5): scores (2.75, -1.25, 1.625, -2.25), max 2.75,
      e = (1, exp(-4) -> 0x1.2c155cp-6, exp(-1.125) -> 0x1.4c71b2p-2, exp(-5) -> 0x1.b993fep-8)
      sum (in order) -> 0x1.598656p+0, inv -> 0x1.7b5784p-1
      prob_3 = e_3 * inv -> 0x1.472a88p-8;  e_3 / sum -> 0x1.472a86p-8."""
    t = [5.5, -2.5, 3.25, -4.5]
    s = [F(F(v) * F(0.5)) for v in t]
    m = max(s)
    e = [expf_cr(F(v - m)) for v in s]
    assert [bits(v) for v in e] == [bits(h(x)) for x in ("0x1p+0", "0x1.2c155cp-6", "0x1.4c71b2p-2",
                                                          "0x1.b993fep-8")]
    total = F(0)
    for v in e:
        total = F(total + v)
    assert bits(total) == bits(h("0x1.598656p+0"))
    inv = F(F(1) / total)
    assert bits(inv) == bits(h("0x1.7b5784p-1"))
    want = [F(v * inv) for v in e]
    assert bits(want[3]) == bits(h("0x1.472a88p-8"))
    got = _attention(orc, 4, t, 4)
    assert [bits(v) for v in got] == [bits(v) for v in want]
    assert bits(F(e[3] / total)) == bits(h("0x1.472a86p-8"))


# ------------------------------------------------------------------ RoPE
def test_rope_rotation_rounds_both_products(orc):
    """rope.rs:514-515, one head of two adjacent pairs, a = 1 + 2^-12, b = 1 + 2^-11:
      pair 0: c = a, s = 1, (x0, x1) = (a, b)
        x0 * c = 1 + 2^-11 + 2^-24: a tie at ulp 2^-23, to even -> b;  x1 * s = b exactly
        x0' = b - b = 0
        x0 * s = a, x1 * c = 1 + 2^-11 + 2^-12 + 2^-23 (exact); x1' = 2 + 2^-10 + 2^-23, a tie
        at ulp 2^-22, to even -> 2 + 2^-10
      pair 1: c = 1, s = a, (x0, x1) = (b, a)
        x0 * c = b exactly;  x1 * s = 1 + 2^-11 + 2^-24 -> b (tie to even);  x0' = 0
        x0 * s = 1 + 2^-11 + 2^-12 + 2^-23 (exact), x1 * c = a; x1' -> 2 + 2^-10 as above.
    Contracting the first product into a fused multiply-add keeps pair 0's exact rounding
    error, x0' = fma(x0, c, -(x1 * s)) = +2^-24; contracting the second keeps pair 1's,
    x0' = fma(-x1, s, x0 * c) = -2^-24.  So either contraction changes a result."""
    a, b = F(1 + 2.0 ** -12), F(1 + 2.0 ** -11)
    cos = np.array([a, 1], F)
    sin = np.array([1, a], F)
    x = np.array([a, b, b, a], F)
    want = [F(0.0), F(2 + 2.0 ** -10), F(0.0), F(2 + 2.0 ** -10)]
    for p in range(2):
        x0, x1, c, s = x[2 * p], x[2 * p + 1], cos[p], sin[p]
        assert bits(F(F(x0 * c) - F(x1 * s))) == bits(want[2 * p])
        assert bits(F(F(x0 * s) + F(x1 * c))) == bits(want[2 * p + 1])
    got = orc.apply_rope(x, 1, 4, 4, cos, sin)
    assert [bits(v) for v in got] == [bits(v) for v in want]
    # pair 0 separates the first contraction, pair 1 the second
    assert bits(fma32(x[0], cos[0], F(-F(x[1] * sin[0])))) == bits(F(2.0 ** -24))
    assert bits(fma32(F(-x[3]), sin[1], F(x[2] * cos[1]))) == bits(F(-(2.0 ** -24)))


def test_rope_frequency_is_powf_of_the_negative_exponent(orc):
    """rope.rs:526-529: theta_i = powf(base, -(i * 2.0) / rope_dim).
      base 500000, rope_dim 128, pair 24: exponent -48/128 = -0.375 (exact);
      500000^-0.375 = 0.0072928...  -> 0x1.ddee9cp-8 (exact value 0.27 ulp above).
      1 / powf(500000, 0.375): 500000^0.375 -> 0x1.123f88p+7, its reciprocal -> 0x1.ddee9ep-8.
      base 10000, rope_dim 96, pair 8: exponent -16/96 -> -0x1.555556p-3 (rounded),
      10000^that -> 0x1.b93a6cp-3; 1 / powf(10000, 0x1.555556p-3) -> 0x1.b93a6ap-3."""
    ex = F(F(-(F(24) * F(2))) / F(128))
    assert float(ex) == -0.375
    want = powf_cr(F(500000.0), ex)
    assert bits(want) == bits(h("0x1.ddee9cp-8"))
    th = orc.rope_frequencies(128, 500000.0)
    assert bits(th[24]) == bits(want)
    assert bits(F(F(1) / powf_cr(F(500000.0), F(0.375)))) == bits(h("0x1.ddee9ep-8"))
    ex2 = F(F(-(F(8) * F(2))) / F(96))
    assert bits(ex2) == bits(h("-0x1.555556p-3"))
    want2 = powf_cr(F(10000.0), ex2)
    assert bits(want2) == bits(h("0x1.b93a6cp-3"))
    th2 = orc.rope_frequencies(96, 10000.0)
    assert bits(th2[8]) == bits(want2)
    assert bits(F(F(1) / powf_cr(F(10000.0), F(-ex2)))) == bits(h("0x1.b93a6ap-3"))
    # every pair of both tables, against the same expression
    for dim, base, table in ((128, 500000.0, th), (96, 10000.0, th2)):
        for i in range(dim // 2):
            e_i = F(F(-(F(i) * F(2))) / F(dim))
            r, dist = correctly_rounded((Decimal(float(e_i)) * Decimal(base).ln()).exp())
            if abs(dist) < 0.3:
                assert bits(table[i]) == bits(r), (dim, i)


def test_llama3_smoothing_association(orc):
    """rope.rs:687-711 in the smoothing band, base 10000, rope_dim 128, factor 40 (not a power
    of two, so where the division sits matters), original context 8192, low 1, high 32:
      pair 47: exponent -94/128 = -0x1.78p-1, f = 10000^that -> 0x1.2eb81cp-10
      wavelength = (2 * PI_f32) / f -> 0x1.54103ap+12 (5441.0) lies in [8192/32, 8192/1]
      smooth = (8192 / wavelength - 1) / (32 - 1) -> 0x1.0b37f8p-6
      ((1 - smooth) * f / 40) + (smooth * f) -> 0x1.8c37d8p-15.
    Each rewrite -- (1 - smooth) * (f / 40), f * ((1 - smooth) / 40 + smooth),
    (f / 40) * (1 - smooth), (1 - smooth) * (f * (1 / 40)) -- gives other bits."""
    f0 = powf_cr(F(10000.0), F(F(-(F(47) * F(2))) / F(128)))
    assert bits(f0) == bits(h("0x1.2eb81cp-10"))
    two_pi = F(F(2) * F(np.pi))
    wl = F(two_pi / f0)
    assert bits(wl) == bits(h("0x1.54103ap+12"))
    orig, low, high, factor = F(8192), F(1), F(32), F(40)
    assert F(orig / high) <= wl <= F(orig / low)
    smooth = F(F(F(orig / wl) - low) / F(high - low))
    assert bits(smooth) == bits(h("0x1.0b37f8p-6"))
    want = F(F(F(F(F(1) - smooth) * f0) / factor) + F(smooth * f0))
    assert bits(want) == bits(h("0x1.8c37d8p-15"))
    th = orc.rope_frequencies(128, 10000.0, 2, 40.0, 8192.0, 1.0, 32.0)
    assert bits(th[47]) == bits(want)
    rewrites = [F(F(F(F(1) - smooth) * F(f0 / factor)) + F(smooth * f0)),
                F(f0 * F(F(F(F(1) - smooth) / factor) + smooth)),
                F(F(F(f0 / factor) * F(F(1) - smooth)) + F(smooth * f0)),
                F(F(F(F(1) - smooth) * F(f0 * F(F(1) / factor))) + F(smooth * f0))]
    assert all(bits(r) != bits(want) for r in rewrites)


# ------------------------------------------------------------------ quantizers
def test_q8_0_quantize_multiplies_by_the_unrounded_inverse(orc):
    """inference.rs:16962-16968: unrounded = amax / 127, inv = 1 / unrounded, q = round(x * inv).
    Block 0: amax = 42.34375 (value 0), unrounded -> 0x1.556ad6p-2, inv -> 0x1.7fe7d0p+1;
      x = -21.171875 = -amax / 2 (value 1): x * inv -> -0x1.fbfffep+5 = -63.4999990... -> -63.
      x / unrounded = -63.5 exactly (unrounded * 63.5 = amax / 2 is exact here), which rounds
      half away from zero to -64.
    Block 1: amax = 1.1171875 (value 0), unrounded = amax / 127 -> 0x1.204082p-7,
      inv -> 0x1.c6b698p+6; x = 0.55859375 = amax / 2: x * inv -> 0x1.fbfffep+5 -> 63.
      With the scale formed as amax * (1 / 127) -> 0x1.204080p-7 (one ulp lower), inv ->
      0x1.c6b69cp+6 and x * inv -> 0x1.fc0002p+5 -> 64."""
    x = np.zeros(64, F)
    x[0], x[1] = 42.34375, -21.171875
    x[32], x[33] = 1.1171875, 0.55859375
    unrounded = F(F(42.34375) / F(127))
    assert bits(unrounded) == bits(h("0x1.556ad6p-2"))
    inv = F(F(1) / unrounded)
    assert bits(inv) == bits(h("0x1.7fe7d0p+1"))
    p = F(x[1] * inv)
    assert bits(p) == bits(h("-0x1.fbfffep+5"))
    assert q8_0_round(p) == -63
    u1 = F(x[32] / F(127))
    assert bits(u1) == bits(h("0x1.204082p-7"))
    inv1 = F(F(1) / u1)
    assert bits(inv1) == bits(h("0x1.c6b698p+6"))
    p1 = F(x[33] * inv1)
    assert bits(p1) == bits(h("0x1.fbfffep+5")) and q8_0_round(p1) == 63
    _, q = orc.quantize_q8_0(x)
    assert [int(v) for v in q[:2]] == [127, -63] and [int(v) for v in q[32:34]] == [127, 63]
    # the rewrites
    assert bits(F(x[1] / unrounded)) == bits(F(-63.5)) and q8_0_round(F(x[1] / unrounded)) == -64
    u2 = F(x[32] * F(F(1) / F(127)))
    assert bits(u2) == bits(h("0x1.204080p-7"))
    assert bits(F(x[33] * F(F(1) / u2))) == bits(h("0x1.fc0002p+5")) and q8_0_round(F(x[33] * F(F(1) / u2))) == 64


def test_q8_k_quantize_iscale_product_and_reciprocal_scale(orc):
    """inference.rs:17584-17590: max = -14.4375 (the signed value of the largest |x|),
      iscale = -127 / max -> 0x1.197d3ap+3 (8.7965...)
      x = 7.21875 = -max / 2: iscale * x -> 0x1.fbfffep+5 = 63.4999990... -> nearest_int 63
  (block value 0 itself maps to -127)
      d = 1 / iscale -> 0x1.d1a348p-4.
    Rewrites: (-127 * x) / max = 63.5 exactly -> nearest_int (ties to even) 64;
    x / (max / -127) -> 63.5 -> 64; d = max / -127 -> 0x1.d1a346p-4."""
    x = np.zeros(256, F)
    x[0], x[1] = -14.4375, 7.21875
    iscale = F(F(-127) / x[0])
    assert bits(iscale) == bits(h("0x1.197d3ap+3"))
    p = F(iscale * x[1])
    assert bits(p) == bits(h("0x1.fbfffep+5"))
    d_want = F(F(1) / iscale)
    assert bits(d_want) == bits(h("0x1.d1a348p-4"))
    d, q = orc.quantize_q8_k(x)
    assert bits(d[0]) == bits(d_want)
    assert int(q[0]) == -127 and int(q[1]) == 63 == orc.nearest_int(float(p))
    assert float(F(F(F(-127) * x[1]) / x[0])) == 63.5 and orc.nearest_int(63.5) == 64
    assert float(F(x[1] / F(x[0] / F(-127)))) == 63.5
    assert bits(F(x[0] / F(-127))) == bits(h("0x1.d1a346p-4")) != bits(d_want)
